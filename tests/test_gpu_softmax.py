"""The retraining model's attention softmax on the device (sf_softmax_rows and its two backward passes,
sparseforge_amd.llama.causal_softmax) against torch's own ops on the same GPU.

The reference's eager attention (legacy/model_llama.py:39-55 under autocast, legacy/main_llama.py:194)
computes p = softmax(scores, dim=-1, dtype=float32).to(scores.dtype) of causal scores (masked entries
-inf), and the Hutchinson HVP (legacy/utils.py:714-869) differentiates its backward once more.  The torch
chain below is that operation with torch's autograd (SoftmaxBackward0, ToCopyBackward0,
SoftmaxBackwardDataBackward0); the device kernels compute the same float32 quantities with another
reduction order and round once to the scores' dtype.

Bar: float32 results within 2e-6 of the output scale (plus 1e-6 relative) elementwise; bf16 results within
one bf16 ulp of torch's (2^-7 relative, an ulp at the bottom of a binade, plus 2^-16 of the output scale: two
float32 computations of one value may round to neighbouring bf16 values); the masked entries exactly 0 in
every output.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _scores(dev, bh, S, dtype, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(bh, S, S, generator=g, device=dev) * 3
    x = x + torch.full((S, S), float("-inf"), device=dev).triu_(1)
    return x.to(dtype)


def _ref(x):
    return torch.softmax(x, dim=-1, dtype=torch.float32).to(x.dtype)


def _close(got, want, dtype):
    got, want = got.float(), want.float()
    scale = want.abs().max().clamp_min(1e-30)
    if dtype == torch.float32:
        bound = 2e-6 * scale + 1e-6 * want.abs()
    else:
        bound = 2.0 ** -7 * want.abs() + 2.0 ** -16 * scale
    return float(((got - want).abs() - bound).max()) <= 0.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("bh,S", [(3, 1), (2, 7), (4, 64), (2, 300), (2, 1024), (2, 2048), (1, 2560)])
def test_forward_backward_double_backward(cuda_device, dtype, bh, S):
    from sparseforge_amd.llama import causal_softmax

    print(f"[softmax] {dtype} bh={bh} S={S}", flush=True)
    x0 = _scores(cuda_device, bh, S, dtype, S)
    g = torch.Generator(device=cuda_device).manual_seed(S + 1)
    gp0 = torch.randn(bh, S, S, generator=g, device=cuda_device).to(dtype)
    ggx = torch.randn(bh, S, S, generator=g, device=cuda_device).to(dtype)
    out = {}
    for name, fn in (("ref", _ref), ("dev", causal_softmax)):
        x = x0.clone().requires_grad_(True)
        gp = gp0.clone().requires_grad_(True)
        p = fn(x)
        (gx,) = torch.autograd.grad(p, x, grad_outputs=gp, create_graph=True)
        gx2, ggp = torch.autograd.grad(gx, (x, gp), grad_outputs=ggx)
        out[name] = (p.detach(), gx.detach(), gx2, ggp)
    masked = torch.ones(S, S, dtype=torch.bool, device=cuda_device).triu_(1)
    for what, a, b in zip(("p", "grad_x", "grad2_x", "grad_grad_p"), out["dev"], out["ref"]):
        assert a.dtype == dtype and a.shape == b.shape, what
        assert not a[:, masked].any(), (what, "masked entries not 0")
        assert _close(a, b, dtype), (what, float((a.float() - b.float()).abs().max()))


def test_rows_past_the_register_capacity_are_refused(cuda_device):
    from sparseforge_amd.llama import causal_softmax

    with pytest.raises(Exception, match="4096"):
        causal_softmax(torch.zeros(1, 4104, 4104, device=cuda_device, dtype=torch.bfloat16))
