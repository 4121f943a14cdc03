"""GPU parity of finalization and the 2:4 packed forward (sf_pack_2to4, sf_unpack_2to4,
sf_gemm_2to4; finalize.finalize_sparse_model / optimize_sparse_model_for_inference /
SparseLinear24).

Bar: packed vals / idx bit-exact against the oracle; unpack(pack(W, M)) == W * M
bit-exact; the sparse-MFMA product elementwise within bf16 rounding
(conftest.gemm_err: 2^-7 of each element plus 2^-12 of the output scale, and the
half ulp of the product that rounding it before the bias adds) of the float64
dense product x . (W * M)^T and of the dense bf16 GEMM of the same weights,
float32 output within 1e-5 of the scale; finalized layers equal the reference's finalization
(mask = hard(soft), weight = W * mask) exactly, and the packed layer's forward
equals the finalized masked layer's within the same bar.
"""
import numpy as np
import pytest
import torch

from conftest import bias_slack, gemm_err
from oracle import masks as om
from oracle import pack24 as op

pytestmark = pytest.mark.gpu


def _mods():
    from sparseforge_amd import finalize as F
    from sparseforge_amd import linear as lin
    from sparseforge_amd import sparse_modeling as sm

    return F, lin, sm


def _wm(out_f, in_f, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(out_f, in_f, generator=g) * 0.05).to(dtype)
    soft = torch.rand(out_f, in_f, generator=g)
    M = torch.from_numpy(om.hard_mask_from_soft(soft.numpy(), "nm_2_4")).to(dtype)
    return W, M


@pytest.mark.parametrize("shape", [(32, 64), (96, 192), (256, 1024)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_pack_matches_oracle_and_round_trips(cuda_device, shape, dtype):
    F, _, _ = _mods()
    W, M = _wm(*shape, seed=shape[0] + shape[1], dtype=dtype)
    M[0, 0:4] = torch.tensor([0, 0, 1, 0], dtype=dtype)  # a group keeping one column
    p = F.pack_2to4(W.to(cuda_device), M.to(cuda_device))
    vals, idx, bad = op.pack(W.float().numpy(), M.float().numpy())
    assert bad == 0
    assert (p.vals.float().cpu().numpy() == op.tile_vals(vals)).all()
    assert (p.idx.cpu().numpy().view(np.uint32) == idx.ravel()).all()
    back = F.unpack_2to4(p, torch.float32).cpu()
    want = torch.from_numpy((W.float() * M.float()).to(torch.bfloat16).float().numpy())
    assert torch.equal(back, want)


def test_pack_rejects_three_of_four(cuda_device):
    F, _, _ = _mods()
    W, M = _wm(32, 64, 3)
    M[4, 8:12] = torch.tensor([1, 1, 1, 0], dtype=M.dtype)
    with pytest.raises(ValueError, match="more than two"):
        F.pack_2to4(W.to(cuda_device), M.to(cuda_device))
    with pytest.raises(ValueError, match="in % 64"):
        F.pack_2to4(W[:, :48].contiguous().to(cuda_device), M[:, :48].contiguous().to(cuda_device))


@pytest.mark.parametrize("tokens,out_f,in_f", [(256, 256, 256), (300, 96, 192), (64, 32, 64), (1000, 768, 1088),
                                               (8192, 4096, 4096)])
@pytest.mark.parametrize("bias", [False, True])
def test_gemm_2to4_matches_dense(cuda_device, tokens, out_f, in_f, bias):
    print(f"[2to4] gemm {tokens}x{out_f}x{in_f} bias={bias}", flush=True)
    F, lin, _ = _mods()
    W, M = _wm(out_f, in_f, seed=tokens + out_f)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(tokens, in_f, generator=g).to(torch.bfloat16)
    b = (torch.randn(out_f, generator=g) * 0.1).to(torch.bfloat16) if bias else None
    d = lambda t: None if t is None else t.to(cuda_device)
    p = F.pack_2to4(d(W), d(M))
    y = F.gemm_2to4(d(x), p, d(b))
    Wm = (W.float() * M.float())
    prod = x.double() @ Wm.double().t()
    ref = prod + b.double() if bias else prod
    # with a bias the product is rounded first, then the sum (as the dense kernel and the reference's
    # out + bias): half an ulp of the product more against the exact value, and against the dense
    # result one ulp (the two float32 sums may round the product to neighbours)
    bf = torch.bfloat16
    assert gemm_err(y, ref, bf, bias_slack(prod, bf) if bias else None) <= 1.0
    dense = lin.mm_nt(d(x), d(Wm.to(torch.bfloat16)), bias=d(b))
    assert gemm_err(y, dense, bf, bias_slack(prod, bf, 1.0) if bias else None) <= 1.0
    y32 = F.gemm_2to4(d(x), p, d(b), out_dtype=torch.float32)
    assert gemm_err(y32, ref, torch.float32) <= 1.0


def _layer(sm, out_f, in_f, dev, slorb=False):
    cfg = sm.SparseLinearConfig(mask_type="structured", hard_mask_type="nm_2_4", SLoRB=slorb, SLoRB_k=16,
                                sparsity_warmup_steps=0)
    layer = sm.SparseLinear(in_f, out_f, sparselinear_config=cfg, bias=True).to(torch.bfloat16).to(dev)
    g = torch.Generator().manual_seed(out_f)
    with torch.no_grad():
        layer.weight.copy_((torch.randn(out_f, in_f, generator=g) * 0.05).to(torch.bfloat16))
        layer.bias.copy_((torch.randn(out_f, generator=g) * 0.1).to(torch.bfloat16))
        layer.mask.copy_(torch.rand(out_f, in_f, generator=g).to(layer.mask.dtype))
        if slorb:
            layer.x_proj.copy_((torch.randn(layer.x_proj.shape, generator=g) * 0.05).to(layer.x_proj.dtype))
            layer.SLoRB_Weight.copy_((torch.randn(layer.SLoRB_Weight.shape, generator=g) * 0.05)
                                     .to(layer.SLoRB_Weight.dtype))
    return layer


def test_finalize_sparse_model_semantics(cuda_device):
    F, _, sm = _mods()
    model = torch.nn.Module()
    model.add_module("a", _layer(sm, 64, 128, cuda_device))
    model.add_module("b", _layer(sm, 32, 64, cuda_device))
    soft = {n: m.mask.detach().float().cpu().numpy() for n, m in model.named_children()}
    W0 = {n: m.weight.detach().float().cpu() for n, m in model.named_children()}
    assert F.finalize_sparse_model(model) == 2
    for n, m in model.named_children():
        hard = om.hard_mask_from_soft(soft[n], "nm_2_4")
        assert (m.mask.detach().float().cpu().numpy() == hard).all()
        want = (W0[n] * torch.from_numpy(hard)).to(torch.bfloat16).float()
        assert torch.equal(m.weight.detach().float().cpu(), want)
        assert m.change_mask is False and m._hardening_finalized is True


@pytest.mark.parametrize("slorb", [False, True])
def test_packed_layer_matches_finalized_forward(cuda_device, slorb):
    F, _, sm = _mods()
    layer = _layer(sm, 256, 512, cuda_device, slorb=slorb)
    model = torch.nn.Module()
    model.add_module("proj", layer)
    F.finalize_sparse_model(model)
    x = torch.randn(4, 100, 512, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(cuda_device)
    with torch.no_grad():
        ref = model.proj(x)
    assert F.convert_model_to_2to4(model, strict=True) == 1
    assert isinstance(model.proj, F.SparseLinear24)
    y = model.proj(x)
    assert y.shape == ref.shape
    # both round x W^T + z S^T (the same z), then add the bias and round again
    slack = bias_slack(ref.float() - model.proj.bias.float(), torch.bfloat16, 1.0)
    assert gemm_err(y, ref, torch.bfloat16, slack) <= 1.0


def test_optimize_for_inference_folds_mask(cuda_device):
    F, _, sm = _mods()
    layer = _layer(sm, 64, 128, cuda_device)
    model = torch.nn.Module()
    model.add_module("l", layer)
    W0 = layer.weight.detach().float().cpu()
    hard = om.hard_mask_from_soft(layer.mask.detach().float().cpu().numpy(), "nm_2_4")
    F.optimize_sparse_model_for_inference(model)
    assert layer.mode == "dense_forward"
    assert torch.equal(layer.weight.detach().float().cpu(), (W0 * torch.from_numpy(hard)).to(torch.bfloat16).float())
