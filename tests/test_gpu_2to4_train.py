"""The hardening_x = 0 training forward on the sparse MFMA (sf_apply_mask_2to4 + sf_gemm_2to4_lowrank).

FusedMaskedLinearSTE.forward (legacy/sparse_modeling.py:56-81) multiplies W by
the effective mask; at hardening_x = 0 with an N:M hard type of 2:4 that mask is
the hard projection (:578-603 / :720-735), which keeps two of every four input
columns, and SparseLinear.forward adds the SLoRB pair (:790-794).  The build
then writes W.E and its packed 2:4 form in one pass and runs the product on
v_smfmac_f32_32x32x32_bf16 with the SLoRB term as a dense second segment.

Bars: the fused pass's W.E is bit-identical to sf_apply_mask's (the input
gradient reuses it) and its packed form to sf_pack_2to4 of W.E; the product is
elementwise within bf16 rounding (conftest.gemm_err: 2^-7 of each element plus
2^-12 of the output scale) of the float64 product and of the dense kernel's
result; through masked_linear the forward matches the dense path within the
same bar and every gradient is bit-identical to it (the backward does not depend
on how y was formed).
"""
import pytest
import torch

from conftest import bias_slack, gemm_err

pytestmark = pytest.mark.gpu


def _mods():
    from sparseforge_amd import _lib as L
    from sparseforge_amd import finalize as F
    from sparseforge_amd import linear as lin

    return L, F, lin


def _mask24(g, out_f, in_f, dev):
    """A byte and-mask keeping two random columns of every group of four."""
    r = torch.rand(out_f, in_f // 4, 4, generator=g, device=dev)
    top = r.topk(2, dim=-1).indices
    m = torch.zeros(out_f, in_f // 4, 4, dtype=torch.uint8, device=dev)
    m.scatter_(-1, top, 255)
    return m.view(out_f, in_f)


def _bits(t):
    return t.view(torch.int16)


@pytest.mark.parametrize("out_f,in_f", [(64, 64), (384, 320), (4096, 4096), (11008, 4096)])
def test_fused_pass_equals_apply_mask_and_pack(cuda_device, out_f, in_f):
    L, F, lin = _mods()
    g = torch.Generator(device=cuda_device).manual_seed(out_f + in_f)
    W = (torch.randn(out_f, in_f, generator=g, device=cuda_device) * 0.02).bfloat16()
    W[0, :8] = torch.tensor([-0.0, 0.0, -1.5, float("nan"), float("inf"), -2.0, 3.0, -0.0], dtype=torch.bfloat16)
    E = _mask24(g, out_f, in_f, cuda_device)
    Wm, vals, idx = lin.apply_mask_2to4(W, E)
    ref = lin.apply_mask(W, E)
    assert torch.equal(_bits(Wm), _bits(ref))
    p = F.pack_2to4(ref, (E != 0).to(torch.bfloat16))
    assert torch.equal(_bits(vals), _bits(p.vals))
    assert torch.equal(idx, p.idx)
    # the packed form holds exactly the kept entries (values compared: unpacking writes a kept -0 as +0)
    back = F.unpack_2to4(F.Packed2to4(vals, idx, out_f, in_f)).float().nan_to_num(7.0)
    assert torch.equal(back, torch.where(E != 0, ref, torch.zeros_like(ref)).float().nan_to_num(7.0))


def _check(got, ref, extra=None):
    err = gemm_err(got, ref, torch.bfloat16, extra)
    assert err <= 1.0, err


@pytest.mark.parametrize("T,out_f,in_f,r,bias", [(1000, 384, 320, 16, True), (8192, 4096, 4096, 64, False),
                                                 (777, 11008, 4096, 64, True), (256, 256, 11008, 0, False)])
def test_lowrank_product(cuda_device, T, out_f, in_f, r, bias):
    L, F, lin = _mods()
    g = torch.Generator(device=cuda_device).manual_seed(T + r)
    x = torch.randn(T, in_f, generator=g, device=cuda_device).bfloat16()
    W = (torch.randn(out_f, in_f, generator=g, device=cuda_device) * 0.02).bfloat16()
    E = _mask24(g, out_f, in_f, cuda_device)
    Wm, vals, idx = lin.apply_mask_2to4(W, E)
    z = S = None
    if r:
        z = torch.randn(T, r, generator=g, device=cuda_device).bfloat16()
        S = (torch.randn(out_f, r, generator=g, device=cuda_device) * 0.05).bfloat16()
    b = (torch.randn(out_f, generator=g, device=cuda_device) * 0.1).bfloat16() if bias else None
    y = lin.gemm_2to4(x, vals, idx, out_f, z=z, S=S, bias=b)
    prod = x.double() @ Wm.double().t()
    if r:
        prod = prod + z.double() @ S.double().t()
    # with a bias the product is rounded first (as the dense kernel and the reference's out + bias):
    # half an ulp of it more against the exact value, one ulp against the dense kernel's result
    bf = torch.bfloat16
    _check(y, prod + b.double() if bias else prod, bias_slack(prod, bf) if bias else None)
    dense = (lin.mm_nt(x, Wm, A2=z, B2=S, K2=r, bias=b) if r else lin.mm_nt(x, Wm, bias=b))
    _check(y, dense.float(), bias_slack(prod, bf, 1.0) if bias else None)


@pytest.mark.parametrize("T,out_f,in_f,r", [(512, 256, 512, 64), (1000, 384, 320, 40)])
def test_masked_linear_hx0_matches_dense_path(cuda_device, T, out_f, in_f, r):
    L, F, lin = _mods()
    g = torch.Generator(device=cuda_device).manual_seed(7 + T)
    x = torch.randn(T, in_f, generator=g, device=cuda_device).bfloat16()
    W = (torch.randn(out_f, in_f, generator=g, device=cuda_device) * 0.02).bfloat16()
    soft = torch.rand(out_f, in_f, generator=g, device=cuda_device)
    P = (torch.randn(r, in_f, generator=g, device=cuda_device) * 0.02).bfloat16()
    S = (torch.randn(out_f, r, generator=g, device=cuda_device) * 0.02).bfloat16()
    gy = torch.randn(T, out_f, generator=g, device=cuda_device).bfloat16()

    def run(force_dense):
        xs, Ws, Ps, Ss = (t.clone().requires_grad_(True) for t in (x, W, P, S))
        if force_dense:
            E = lin.effective_mask(soft, torch.uint8, "hard", 0.0, L.HARD_NM_TAIL_KEEP, 2, 4)
            Pp, Sp = (Ps, Ss)
            if r % 8:
                Pp, Sp, _ = lin._PadRank.apply(Ps, Ss)
            y = lin._MaskedLinear.apply(xs, Ws, None, Pp, Sp, E, 1.0, 0.0, False)
        else:
            y = lin.masked_linear(xs, Ws, None, soft, "mix", 0.0, L.HARD_NM_TAIL_KEEP, 2, 1.0, Ps, Ss)
        y.backward(gy)
        return y.detach(), xs.grad, Ws.grad, Ps.grad, Ss.grad

    y24, *g24 = run(False)
    yd, *gd = run(True)
    _check(y24, yd.float())
    for a, b in zip(g24, gd):
        assert torch.equal(_bits(a), _bits(b))


def test_sparselinear_hx0_uses_the_sparse_product(cuda_device):
    """SparseLinear at hardening_x = 0 with nm_2_4 goes through sf_gemm_2to4_lowrank."""
    from sparseforge_amd import profiling as prof
    from sparseforge_amd import sparse_modeling as sm

    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="nm_2_4", SLoRB=True, SLoRB_k=64,
                                sparsity_warmup_steps=0)
    m = sm.SparseLinear(512, 256, sparselinear_config=cfg, bias=False, device=cuda_device).to(torch.bfloat16)
    m.hardening_x = 0.0
    x = torch.randn(4, 64, 512, device=cuda_device).bfloat16()
    with prof.kernel_timer() as t:
        y = m(x)
    names = set(t.summary())
    assert "sf_gemm_2to4" in names and "sf_apply_mask_2to4" in names, names
    assert y.shape == (4, 64, 256)
