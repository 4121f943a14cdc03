"""The retraining model's gated MLP product on the device (sf_swiglu_forward / _backward / _double_backward):
silu(gate) * up, as HuggingFace's LlamaMLP computes it, against torch's ops.

Bars: forward and backward against F.silu(g) * u with torch's autograd on the same inputs -- f32 within 1e-6
relative, bf16 within one bf16 rounding (the kernels evaluate torch's silu, mul and silu_backward formulas and
round where torch rounds; exp may differ from torch's by an ulp); the double backward (closed form in f32)
against float64 autograd of the same map on the same values: f32 within 1e-5 relative (norm-wise), bf16 within
the final rounding (1e-2), for probes on either output or both.
"""
import pytest
import torch
from torch.nn import functional as F

pytestmark = pytest.mark.gpu


def _close(a, b, dtype):
    a, b = a.float(), b.float()
    if dtype == torch.float32:
        assert torch.allclose(a, b, rtol=1e-6, atol=1e-6), float((a - b).abs().max())
    else:
        tol = b.abs().clamp_min(a.abs()) * 2.0 ** -7 + 1e-6
        assert bool(((a - b).abs() <= tol).all()), float(((a - b).abs() / tol).max())


def _inputs(shape, dtype, dev, seed):
    gen = torch.Generator(device=dev).manual_seed(seed)
    mk = lambda s: (torch.randn(shape, generator=gen, device=dev) * s).to(dtype)  # noqa: E731
    return mk(3.0), mk(1.0), mk(1.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(64, 5632), (3, 8), (17, 96)])
def test_forward_backward_match_torch(cuda_device, dtype, shape):
    from sparseforge_amd import llama

    print(f"[swiglu] fwd/bwd {shape} {dtype}", flush=True)
    g0, u0, gy = _inputs(shape, dtype, cuda_device, sum(shape))
    g0.view(-1)[:4] = torch.tensor([0.0, -90.0, 90.0, -0.0], device=cuda_device).to(dtype)  # exp limits
    outs = []
    for fn in (llama.swiglu, lambda g, u: F.silu(g) * u):
        g, u = g0.clone().requires_grad_(True), u0.clone().requires_grad_(True)
        y = fn(g, u)
        outs.append((y,) + torch.autograd.grad(y, (g, u), gy))
    for a, b in zip(*outs):
        assert a.dtype == dtype
        _close(a, b, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("probe", ["both", "gate", "up"])
def test_double_backward_matches_float64_autograd(cuda_device, dtype, probe):
    from sparseforge_amd import llama

    print(f"[swiglu] double backward {dtype} {probe}", flush=True)
    g0, u0, gy0 = _inputs((40, 520), dtype, cuda_device, 11)
    gen = torch.Generator(device=cuda_device).manual_seed(3)
    pg = torch.randn(40, 520, generator=gen, device=cuda_device).to(dtype)
    pu = torch.randn(40, 520, generator=gen, device=cuda_device).to(dtype)

    def hvp(fn, g0, u0, gy0):
        g, u, gy = (t.clone().requires_grad_(True) for t in (g0, u0, gy0))
        y = fn(g, u)
        gg, gu = torch.autograd.grad(y, (g, u), gy, create_graph=True)
        dot = 0.0
        if probe in ("both", "gate"):
            dot = dot + (gg.double() * pg.double()).sum()
        if probe in ("both", "up"):
            dot = dot + (gu.double() * pu.double()).sum()
        return torch.autograd.grad(dot, (g, u, gy), allow_unused=True)

    got = hvp(llama.swiglu, g0, u0, gy0)
    ref = hvp(lambda g, u: F.silu(g) * u, g0.double(), u0.double(), gy0.double())
    bar = 1e-5 if dtype == torch.float32 else 1e-2
    for a, b in zip(got, ref):
        if b is None:
            assert a is None or float(a.abs().max()) == 0.0
            continue
        err = float((a.double() - b).norm() / b.norm().clamp_min(1e-30))
        assert err < bar, err


def test_swiglu_dispatch_and_bad_calls(cuda_device):
    from sparseforge_amd import _lib as L
    from sparseforge_amd import llama

    g = torch.randn(4, 16, device=cuda_device).to(torch.bfloat16).requires_grad_(True)
    u = torch.randn(4, 16, device=cuda_device).to(torch.bfloat16)
    assert llama.swiglu(g, u).grad_fn.__class__.__name__ == "_SwiGLUBackward"
    odd = torch.randn(3, 5, device=cuda_device).to(torch.bfloat16)  # 15 elements: torch's ops
    assert llama.swiglu(odd.requires_grad_(True), odd.detach()).grad_fn.__class__.__name__ == "MulBackward0"
    lib, st = L.lib(), L.stream(cuda_device)
    x = torch.empty(64, device=cuda_device)
    assert lib.sf_swiglu_forward(L.ptr(x), L.ptr(x), L.DT_F32, 12, L.ptr(x), st) == L.SF_ERR_INVALID
    assert lib.sf_swiglu_forward(L.ptr(x) + 4, L.ptr(x), L.DT_F32, 8, L.ptr(x), st) == L.SF_ERR_INVALID
    assert lib.sf_swiglu_forward(L.ptr(x), L.ptr(x), 7, 8, L.ptr(x), st) == L.SF_ERR_INVALID
