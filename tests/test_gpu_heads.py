"""Per-head attention operands on the device (sf_to_heads / sf_from_heads) against torch's layout ops.

The retraining model's attention follows HuggingFace's eager LlamaAttention (legacy/model_llama.py:39-55):
q, k, v views [B, S, H, D] transposed to [B, H, S, D], the half-split rotary embedding on q and k in the
activations' dtype, per-head products.  llama._causal_attention_torch writes it with torch's transposes,
rolls and products (the CPU path, pinned to transformers.LlamaForCausalLM in
tests/test_llama_reference_model.py); on the GPU the model runs llama._causal_attention_device, whose
layout changes and rotation are one kernel pass each way.  Bar: bit-exact in bf16 and f32 -- the kernels
round each product and then the sum to the dtype, as torch's ops do -- for the forward, the backward and
the double backward that the Hutchinson probe takes, and for the kernels alone (both layouts, partial
position tiles, head dims 16 to 128).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _tables(S, D, dev):
    from sparseforge_amd import llama

    return llama.rotary_tables(S, D, 10000.0, dev)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,S,H,D", [(2, 128, 4, 64), (1, 100, 3, 16), (2, 72, 2, 128), (3, 64, 5, 32)])
def test_to_heads_and_adjoint_match_torch(cuda_device, dtype, B, S, H, D):
    from sparseforge_amd import llama

    g = torch.Generator(device=cuda_device).manual_seed(B * 1000 + S + D)
    x = torch.randn(B, S, H, D, generator=g, device=cuda_device).to(dtype)
    cos, sin = _tables(S, D, cuda_device)
    c, s_ = cos.to(dtype), sin.to(dtype)
    for rotate in (True, False):
        for scale in (1.0, 0.125):
            ref = (llama._rotate(x.transpose(1, 2), c, s_) if rotate else x.transpose(1, 2)) * scale
            ref = ref.reshape(B * H, S, D)
            xr = x.clone().requires_grad_(True)
            y = llama._ToHeads.apply(xr, cos, sin, rotate, False, scale)
            assert torch.equal(y, ref), (rotate, scale)
            yt = llama._ToHeads.apply(x, cos, sin, rotate, True, scale)
            assert torch.equal(yt, ref.transpose(1, 2)), (rotate, scale)
            # the adjoint against torch's gradient of the same map
            gy = torch.randn(B * H, S, D, generator=g, device=cuda_device).to(dtype)
            xt = x.clone().requires_grad_(True)
            yy = (llama._rotate(xt.transpose(1, 2), c, s_) if rotate else xt.transpose(1, 2)) * scale
            (gref,) = torch.autograd.grad(yy.reshape(B * H, S, D), xt, gy)
            (gx,) = torch.autograd.grad(y, xr, gy)
            assert torch.equal(gx, gref), (rotate, scale)
            # the transposed layout's adjoint, from a contiguous [B H, D, S] gradient and from a transposed view
            gxt = llama._FromHeads.apply(gy.transpose(1, 2).contiguous(), cos, sin, (B, S, H, D), rotate, True,
                                         scale)
            assert torch.equal(gxt, gref)
            gxv = llama._FromHeads.apply(gy.transpose(1, 2), cos, sin, (B, S, H, D), rotate, True, scale)
            assert torch.equal(gxv, gref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("S,D", [(192, 64), (160, 96)])
def test_device_attention_matches_torch_form(cuda_device, dtype, S, D):
    """Forward, backward and the Hutchinson double backward of causal_attention: the device path (plain
    score product, the causal softmax masking the tail itself) equals the torch form (the score product
    plus the -inf mask) bit for bit; D = 96 takes the scale after the product (96^-0.5 is not a power of
    two)."""
    from sparseforge_amd import llama

    B, H = 2, 4
    g = torch.Generator(device=cuda_device).manual_seed(7)
    mk = lambda: (torch.randn(B, S, H, D, generator=g, device=cuda_device) * 0.5).to(dtype)  # noqa: E731
    q0, k0, v0 = mk(), mk(), mk()
    w = torch.randn(B, S, H * D, generator=g, device=cuda_device).to(dtype)
    probes = [torch.randn(B, S, H, D, generator=g, device=cuda_device).to(dtype) for _ in range(3)]
    cos, sin = _tables(S, D, cuda_device)
    outs = []
    for fn in (llama._causal_attention_torch, llama._causal_attention_device):
        q, k, v = (t.clone().requires_grad_(True) for t in (q0, k0, v0))
        y = fn(q, k, v, cos, sin)
        loss = (y.float() * w.float()).sum()
        grads = torch.autograd.grad(loss, (q, k, v), create_graph=True)
        dot = sum((gr.float() * p.float()).sum() for gr, p in zip(grads, probes))
        hv = torch.autograd.grad(dot, (q, k, v))
        outs.append((y.detach(), [gr.detach() for gr in grads], hv))
    (y0, g0, h0), (y1, g1, h1) = outs
    assert torch.equal(y1, y0)
    for a, b in zip(g1, g0):
        assert torch.equal(a, b)
    for a, b in zip(h1, h0):
        assert torch.equal(a, b)


def test_heads_reject_bad_calls(cuda_device):
    from sparseforge_amd import _lib as L

    x = torch.zeros(2, 8, 2, 64, device=cuda_device)
    y = torch.empty(4, 8, 64, device=cuda_device)
    cos, sin = _tables(8, 64, cuda_device)
    lib = L.lib()
    st = L.stream(cuda_device)
    assert lib.sf_to_heads(L.ptr(x), L.DT_F32, 2, 8, 2, 24, L.ptr(cos), L.ptr(sin), 1, 0, 1.0, L.ptr(y), st) \
        == L.SF_ERR_INVALID  # head dim not a multiple of 16
    assert lib.sf_to_heads(L.ptr(x), L.DT_F32, 2, 8, 2, 64, None, None, 1, 0, 1.0, L.ptr(y), st) == L.SF_ERR_INVALID
    assert lib.sf_from_heads(L.ptr(y), 9, 2, 8, 2, 64, L.ptr(cos), L.ptr(sin), 0, 0, 1.0, L.ptr(x), st) \
        == L.SF_ERR_INVALID


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(3, 128, 192), (2, 100, 72), (1, 7, 130), (4, 64, 64)])
def test_transpose_batched(cuda_device, dtype, shape):
    """The derivatives' transposed operands (llama._contig3 -> sf_transpose_batched): exactly torch's
    contiguous copy of the transposed view, whole and partial 64 x 64 tiles, rows / cols not multiples of 8."""
    from sparseforge_amd import llama

    g = torch.Generator(device=cuda_device).manual_seed(sum(shape))
    x = torch.randn(shape, generator=g, device=cuda_device).to(dtype)
    got = llama._contig3(x.transpose(1, 2))
    assert got.is_contiguous() and torch.equal(got, x.transpose(1, 2).contiguous())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_device_attention_causal_blocks(cuda_device, dtype):
    """At S >= 512 the device path's attention products run as causal blocks (llama._CBMM: only the blocks
    the lower triangle touches); forward, backward and the Hutchinson double backward against the torch
    form's full products: f32 within 1e-4, bf16 within 2e-2 (norm-wise relative; the blocks accumulate in
    another order than the full products, and bf16 rounds each operand)."""
    from sparseforge_amd import llama

    B, S, H, D = 1, 1024, 4, 64
    g = torch.Generator(device=cuda_device).manual_seed(11)
    mk = lambda: (torch.randn(B, S, H, D, generator=g, device=cuda_device) * 0.5).to(dtype)  # noqa: E731
    q0, k0, v0 = mk(), mk(), mk()
    w = torch.randn(B, S, H * D, generator=g, device=cuda_device).to(dtype)
    probes = [torch.randn(B, S, H, D, generator=g, device=cuda_device).to(dtype) for _ in range(3)]
    cos, sin = _tables(S, D, cuda_device)
    outs = []
    for fn in (llama._causal_attention_device, llama._causal_attention_torch):
        q, k, v = (t.clone().requires_grad_(True) for t in (q0, k0, v0))
        y = fn(q, k, v, cos, sin)
        loss = (y.float() * w.float()).sum()
        grads = torch.autograd.grad(loss, (q, k, v), create_graph=True)
        dot = sum((gr.float() * p.float()).sum() for gr, p in zip(grads, probes))
        hv = torch.autograd.grad(dot, (q, k, v))
        outs.append([y.detach()] + [gr.detach() for gr in grads] + list(hv))
    bar = 1e-4 if dtype == torch.float32 else 2e-2
    for a, b in zip(*outs):
        assert torch.isfinite(a).all()
        err = float((a.double() - b.double()).norm() / b.double().norm())
        assert err < bar, err
