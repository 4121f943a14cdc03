"""RMSNorm of the retraining model on the device (sf_rmsnorm_forward / _backward / _double_backward) against
torch's ops.

The reference retrains HuggingFace's LlamaForCausalLM, whose LlamaRMSNorm is
weight * (x32 * rsqrt(mean(x32^2) + eps)).to(x dtype) (llama.rms_norm_torch writes the same ops; it is pinned
to transformers in tests/test_llama_reference_model.py), and the Hutchinson probe differentiates its backward
once more.  Bars:
* forward and backward against the torch form on the same inputs: f32 within 1e-5 relative (the row sums run
  in another order); bf16 within one bf16 rounding of the torch form's value (the kernels round where torch's
  ops round, so only an f32-level difference that crosses a rounding boundary shows);
* the double backward (the closed-form derivatives in f32) against torch's autograd of the torch form in
  float64 on the same values: f32 inputs within 1e-4 relative (norm-wise), bf16 inputs within the final bf16
  rounding (1e-2 norm-wise), with and without a weight-gradient term in the probe.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [(64, 2048), (33, 96), (5, 4096), (7, 8), (300, 520)]


def _inputs(rows, D, dtype, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = (torch.randn(rows, D, generator=g, device=dev) * 1.5).to(dtype)
    w = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(dtype)
    gy = torch.randn(rows, D, generator=g, device=dev).to(dtype)
    return x, w, gy


def _close_dtype(a, b, dtype):
    a, b = a.float(), b.float()
    if dtype == torch.float32:
        assert torch.allclose(a, b, rtol=1e-5, atol=1e-5), float((a - b).abs().max())
    else:  # one bf16 step of the larger magnitude
        tol = b.abs().clamp_min(a.abs()) * 2.0 ** -7 + 1e-6
        assert bool(((a - b).abs() <= tol).all()), float(((a - b).abs() / tol).max())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", SHAPES)
def test_forward_backward_match_torch(cuda_device, dtype, shape):
    from sparseforge_amd import llama

    rows, D = shape
    print(f"[norm] fwd/bwd {shape} {dtype}", flush=True)
    x0, w0, gy = _inputs(rows, D, dtype, cuda_device, rows * 7 + D)
    outs = []
    for dev_path in (True, False):
        x, w = x0.clone().requires_grad_(True), w0.clone().requires_grad_(True)
        if dev_path:
            y = llama._RMSNorm.apply(x, w, 1e-5)
        else:
            y = llama.rms_norm_torch(x, w, 1e-5)
        gx, gw = torch.autograd.grad(y, (x, w), gy)
        outs.append((y, gx, gw))
    (y1, gx1, gw1), (y0, gx0, gw0) = outs
    assert y1.dtype == dtype and gx1.dtype == dtype and gw1.dtype == dtype
    _close_dtype(y1, y0, dtype)
    _close_dtype(gx1, gx0, dtype)
    # the weight gradient sums rows of rounded products: f32 order differences over up to 300 rows
    a, b = gw1.float(), gw0.float()
    scale = (gy.float().abs() * 3.0).sum(0) * (2.0 ** -20 if dtype == torch.float32 else 2.0 ** -7)
    assert bool(((a - b).abs() <= scale + b.abs() * 2.0 ** -7).all())


def _hvp(norm, x0, w0, gy, px, pw, with_w):
    x, w = x0.clone().requires_grad_(True), w0.clone().requires_grad_(True)
    y = norm(x, w)
    gx, gw = torch.autograd.grad(y, (x, w), gy, create_graph=True)
    dot = (gx.double() * px.double()).sum()
    if with_w:
        dot = dot + (gw.double() * pw.double()).sum()
    return torch.autograd.grad(dot, (x, w), allow_unused=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("with_w", [True, False])
@pytest.mark.parametrize("shape", [(64, 2048), (33, 96), (5, 4096)])
def test_double_backward_matches_float64_autograd(cuda_device, dtype, with_w, shape):
    from sparseforge_amd import llama

    rows, D = shape
    print(f"[norm] double backward {shape} {dtype} with_w={with_w}", flush=True)
    x0, w0, gy = _inputs(rows, D, dtype, cuda_device, rows + 3 * D)
    g = torch.Generator(device=cuda_device).manual_seed(5)
    px = torch.randn(rows, D, generator=g, device=cuda_device).to(dtype)
    pw = torch.randn(D, generator=g, device=cuda_device).to(dtype)
    hx, hw = _hvp(lambda x, w: llama._RMSNorm.apply(x, w, 1e-5), x0, w0, gy, px, pw, with_w)
    # float64 autograd of the same map on the same values (no intermediate rounding)
    def ref(x, w):
        return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5))

    rx, rw = _hvp(ref, x0.double(), w0.double(), gy.double(), px.double(), pw.double(), with_w)
    bar = 1e-4 if dtype == torch.float32 else 1e-2
    for got, ref in ((hx, rx), (hw, rw)):
        err = float((got.double() - ref).norm() / ref.norm().clamp_min(1e-30))
        assert err < bar, err


def test_model_norm_dispatch(cuda_device):
    """RMSNorm modules take the device passes for eligible inputs and torch's ops otherwise."""
    from sparseforge_amd import llama

    def device_node(t):  # the output view's producer
        fn = t.grad_fn
        if fn.__class__.__name__ == "ViewBackward0":
            fn = fn.next_functions[0][0]
        return fn.__class__.__name__.startswith("_RMSNorm")

    m = llama.RMSNorm(96, 1e-5, device=cuda_device, dtype=torch.bfloat16)
    x = torch.randn(4, 10, 96, device=cuda_device).to(torch.bfloat16).requires_grad_(True)
    y = m(x)
    assert y.shape == x.shape and device_node(y)
    _close_dtype(y, llama.rms_norm_torch(x, m.weight, 1e-5), torch.bfloat16)
    odd = llama.RMSNorm(12, 1e-5, device=cuda_device, dtype=torch.bfloat16)  # 12 % 8 != 0: torch's ops
    z = odd(torch.randn(3, 12, device=cuda_device).to(torch.bfloat16))
    assert not device_node(z)


def test_norm_rejects_bad_calls(cuda_device):
    from sparseforge_amd import _lib as L

    x = torch.zeros(4, 8192, device=cuda_device)
    w = torch.ones(8192, device=cuda_device)
    r = torch.empty(4, device=cuda_device)
    lib, st = L.lib(), L.stream(cuda_device)
    assert lib.sf_rmsnorm_forward(L.ptr(x), L.ptr(w), L.DT_F32, 4, 8192, 1e-5, L.ptr(x), L.ptr(r), st) \
        == L.SF_ERR_INVALID  # longer than 4096
    assert lib.sf_rmsnorm_forward(L.ptr(x), L.ptr(w), L.DT_F32, 4, 12, 1e-5, L.ptr(x), L.ptr(r), st) \
        == L.SF_ERR_INVALID  # not a multiple of 8
    assert lib.sf_rmsnorm_forward(L.ptr(x) + 4, L.ptr(w), L.DT_F32, 4, 8, 1e-5, L.ptr(x), L.ptr(r), st) \
        == L.SF_ERR_INVALID  # misaligned
    ws = torch.empty(16, dtype=torch.uint8, device=cuda_device)
    assert lib.sf_rmsnorm_backward(L.ptr(x), L.ptr(w), L.ptr(x), L.ptr(r), L.DT_F32, 4, 2048, L.ptr(x), L.ptr(w),
                                   L.ptr(ws), 16, st) == L.SF_ERR_INVALID  # workspace too small
