"""GPU parity of the block hard types and block_sparse masks (sf_block_stat, sf_topk_keep,
sf_tile_topk, sf_block_fill, sf_apply_gate, sf_freeze_mask, sf_effective_mask_given).

Bar: hard masks, targets and flip counts bit-exact against the reference's own outputs
(tests/golden/ref_hardblk_*, ref_updblk_*) and the oracle; f32 G and soft masks within 1e-6;
block statistics within a few f32 ulp (exact for blocks of equal elements).
"""
import ast

import numpy as np
import pytest
import torch

from conftest import load_golden
from oracle import masks as om

pytestmark = pytest.mark.gpu


def _mods():
    from sparseforge_amd import _lib as L
    from sparseforge_amd import kernels as K
    from sparseforge_amd import sparse_modeling as sm

    return L, K, sm


def _layer(r, kw, dev, dtype=torch.float32):
    _, _, sm = _mods()
    cfg = sm.SparseLinearConfig(**kw)
    if kw.get("mask_metric", "") in ("hessian_ratio", "hessian_obd", "hessian"):
        cfg.enable_hutchinson = True
    W = r["W"]
    layer = sm.SparseLinear(W.shape[1], W.shape[0], sparselinear_config=cfg, bias=False).to(dtype).to(dev)
    with torch.no_grad():
        layer.weight.copy_(torch.from_numpy(W))
        if not layer._is_placeholder("hessian_diag"):
            layer.hessian_diag.copy_(torch.from_numpy(r["H"]))
    return layer


@pytest.mark.parametrize("case", ["hardblk_block16_f32", "hardblk_block16_sr03_f32", "hardblk_block16_ones_f32",
                                  "hardblk_bs16_f32", "hardblk_bs16_sr03_f32", "hardblk_bs16_ones_f32",
                                  "hardblk_bs32_f32"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_hard_mask_matches_reference(cuda_device, case, dtype):
    _, _, sm = _mods()
    r = load_golden(case)
    soft = torch.from_numpy(r["soft"]).to(dtype)
    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type=str(r["hard_type"]),
                                sparsity_ratio=float(r["sr"]))
    layer = sm.SparseLinear(soft.shape[1], soft.shape[0], sparselinear_config=cfg, bias=False).to(cuda_device)
    got = layer._hard_mask_from_soft(soft.to(cuda_device))
    assert got.dtype == dtype
    ref = r["hard"] if dtype == torch.float32 else om.hard_mask_from_soft(
        soft.float().numpy(), str(r["hard_type"]), sparsity_ratio=float(r["sr"]))
    assert np.array_equal(got.float().cpu().numpy(), ref)


def _torch_keep(v, k):
    """The entries torch.topk keeps (CPU kernel) as a boolean mask along the last axis."""
    t = torch.from_numpy(np.ascontiguousarray(v))
    keep = torch.zeros(t.shape, dtype=torch.bool)
    if k > 0:
        keep.scatter_(-1, torch.topk(t, k, dim=-1).indices, True)
    return keep.numpy()


@pytest.mark.parametrize("n, k, nv", [(1, 1, 50), (7, 3, 2), (1000, 0, 50), (1000, 1000, 50), (1000, 999, 50),
                                      (176128, 88064, 50), (176128, 88064, 3), (44032, 13210, 2), (300001, 12345, 50),
                                      (300001, 4000, 50), (5000, 70, 4), (256, 1, 3), (9, 9 // 2, 1)])
def test_topk_keep_matches_torch_with_ties(cuda_device, n, k, nv):
    """Equal values kept exactly as torch.topk keeps them, on both sides of its partial-sort switch."""
    _, K, _ = _mods()
    rng = np.random.default_rng(n + k + nv)
    v = rng.integers(0, nv, size=n).astype(np.float32) / 7.0  # heavy ties
    if n > 10:
        v[rng.integers(0, n, size=3)] = np.nan
        v[rng.integers(0, n, size=3)] = -0.0
    got = K.topk_keep(torch.from_numpy(v).to(cuda_device), k).cpu().numpy() > 0.5
    assert np.array_equal(got, om.topk_keep_desc(v, k))
    if 0 < k < n:
        assert np.array_equal(got, _torch_keep(v, k))


@pytest.mark.parametrize("shape, k", [((64, 96), 128), ((40, 56), 179), ((33, 50), 1), ((48, 48), 255),
                                      ((32, 32), 0), ((32, 32), 256), ((1024, 4096), 128), ((256, 512), 4),
                                      ((256, 512), 3)])
def test_tile_topk_matches_oracle_with_ties(cuda_device, shape, k):
    _, K, _ = _mods()
    rng = np.random.default_rng(shape[0] + k)
    x = (rng.integers(0, 20, size=shape) / 19.0).astype(np.float32)
    got = K.tile_topk(torch.from_numpy(x).to(cuda_device), k, torch.float32).cpu().numpy()
    sr = 1.0 - k / 256.0
    assert om.keep_count(1.0 - sr, 256) == k
    assert np.array_equal(got, om.hard_mask_from_soft(x, "block16", sparsity_ratio=sr))
    if 0 < k < 256:  # against torch.topk along each flattened tile
        of, inf = shape[0] // 16 * 16, shape[1] // 16 * 16
        ob, ib = of // 16, inf // 16
        tiles = x[:of, :inf].reshape(ob, 16, ib, 16).transpose(0, 2, 1, 3).reshape(ob, ib, 256)
        want = _torch_keep(tiles, k).reshape(ob, ib, 16, 16).transpose(0, 2, 1, 3).reshape(of, inf)
        assert np.array_equal(got[:of, :inf] > 0.5, want)


@pytest.mark.parametrize("bs", [16, 32])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_stat_matches_oracle(cuda_device, bs, dtype):
    L, K, _ = _mods()
    rng = np.random.default_rng(bs)
    x = torch.from_numpy(rng.standard_normal((200, 330)).astype(np.float32)).to(dtype)
    x[:bs, :bs] = 0.375  # a constant block: exact
    xf = x.float().numpy()
    xd = x.to(cuda_device)
    mean = K.block_stat(xd, bs, L.BLOCK_MEAN).cpu().numpy()
    rms = K.block_stat(xd, bs, L.BLOCK_RMS).cpu().numpy()
    np.testing.assert_allclose(mean, om.block_mean(xf, bs).ravel(), rtol=0, atol=1e-7)
    np.testing.assert_allclose(rms, om.block_rms(xf, bs).ravel(), rtol=2e-7, atol=0)
    assert mean[0] == np.float32(0.375) and rms[0] == np.float32(0.375)


def test_blockify_keeps_edges(cuda_device):
    _, _, sm = _mods()
    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="block_sparse16")
    layer = sm.SparseLinear(70, 50, sparselinear_config=cfg, bias=False).to(cuda_device)
    t = torch.rand(50, 70, generator=torch.Generator().manual_seed(2))
    got = layer._blockify_tensor(t.to(cuda_device)).cpu().numpy()
    np.testing.assert_allclose(got, om.blockify(t.numpy(), "block_sparse16", "f32"), rtol=0, atol=1e-7)
    assert np.array_equal(got[48:], t.numpy()[48:]) and np.array_equal(got[:, 64:], t.numpy()[:, 64:])


@pytest.mark.parametrize("case", ["gateblk_bs16_f32", "gateblk_bs32_struct_f32", "gateblk_bs16_small_f32"])
def test_block_gate_matches_reference(cuda_device, case):
    r = load_golden(case)
    kw = ast.literal_eval(str(r["cfg"]))
    layer = _layer(r, kw, cuda_device)
    with torch.no_grad():
        layer.mask.copy_(torch.from_numpy(r["mask"]))
        if not layer._is_placeholder("frozen_mask_flags"):
            layer.frozen_mask_flags.copy_(torch.from_numpy(r["frozen"]))
    idx = torch.from_numpy(r["idx"]).to(cuda_device)
    n = r["W"].size
    G = layer.compute_gate_target(int(r["step"]), sample_idx=idx if idx.numel() < n else None)
    np.testing.assert_allclose(G.cpu().numpy(), r["G"], rtol=0, atol=1e-6)


@pytest.mark.parametrize("case", ["updblk_bs16_f32", "updblk_block16_pen_f32", "updblk_bs32_freeze_f32",
                                  "updblk_block16_hard_f32"])
def test_block_update_matches_reference(cuda_device, case):
    r = load_golden(case)
    kw = ast.literal_eval(str(r["cfg"]))
    layer = _layer(r, kw, cuda_device)
    has_frozen = not layer._is_placeholder("frozen_mask_flags")
    with torch.no_grad():
        layer.mask.copy_(torch.from_numpy(r["init_mask"]))
        if has_frozen:
            layer.frozen_mask_flags.copy_(torch.from_numpy(r["init_frozen"]))
    n = r["W"].size
    for j, step in enumerate(r["steps"]):
        idx = torch.from_numpy(r[f"idx{j}"]).to(cuda_device)
        layer.update_mask(int(step), lambda_mid=float(r["lam"]), sample_idx=idx if idx.numel() < n else None)
        np.testing.assert_allclose(layer.mask.cpu().numpy(), r[f"mask{j}"], rtol=0, atol=1e-6)
        assert int(layer.weight.flipped_mask) == int(r[f"flips{j}"])
        assert layer.hardening_x == float(r[f"hx{j}"])
        if has_frozen:
            assert np.array_equal(layer.frozen_mask_flags.cpu().numpy(), r[f"frozen{j}"])
        with torch.no_grad():
            layer.mask.copy_(torch.from_numpy(r[f"mask{j}"]))


@pytest.mark.parametrize("hard_type, pen", [("block_sparse16", "block_sparse16"), ("block_sparse32", "mid"),
                                            ("block16", "block16")])
def test_block_update_larger_matches_oracle(cuda_device, hard_type, pen):
    """[520, 800] (a ragged core, many blocks) against the oracle, one step."""
    _, _, sm = _mods()
    kw = dict(mask_type="unstructured", hard_mask_type=hard_type, mask_metric="hessian_ratio",
              sparsity_warmup_steps=0, mask_update_period=1, mask_penalty_mode=pen, mask_penalty_lr=0.1,
              mask_binarize_decay=0.02, mask_lr=0.2, tau_sample_size=4096)
    rows, cols = 520, 800
    g = torch.Generator().manual_seed(len(hard_type) + len(pen))
    W = torch.randn(rows, cols, generator=g) * 0.02
    H = torch.rand(rows, cols, generator=g) * 1e-3 + 1e-6
    M0 = torch.rand(rows, cols, generator=g)
    cfg = sm.SparseLinearConfig(**kw)
    cfg.enable_hutchinson = True
    layer = sm.SparseLinear(cols, rows, sparselinear_config=cfg, bias=False).to(cuda_device)
    with torch.no_grad():
        layer.weight.copy_(W)
        layer.hessian_diag.copy_(H)
        layer.mask.copy_(M0)
    idx = torch.randint(0, rows * cols, (4096,), generator=g)
    layer.update_mask(5, lambda_mid=0.2, sample_idx=idx.to(cuda_device))
    new, _, flips, _ = om.layer_update_mask(om.full_config(**kw), 5, W.numpy(), H.numpy(), M0.numpy(), None,
                                            idx.numpy(), 0.2)
    np.testing.assert_allclose(layer.mask.cpu().numpy(), new, rtol=0, atol=1e-6)
    assert int(layer.weight.flipped_mask) == flips


def test_block_sparse_forward_mix(cuda_device):
    """E = hx soft + (1 - hx) hard(soft) with the whole-tensor block_sparse16 projection, through the GEMM."""
    _, _, sm = _mods()
    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="block_sparse16")
    layer = sm.SparseLinear(96, 80, sparselinear_config=cfg, bias=False).to(cuda_device)
    g = torch.Generator().manual_seed(4)
    W = torch.randn(80, 96, generator=g) * 0.05
    M = torch.rand(80, 96, generator=g)
    x = torch.randn(37, 96, generator=g)
    with torch.no_grad():
        layer.weight.copy_(W)
        layer.mask.copy_(M)
    for hx in (0.3, 0.0):
        layer.hardening_x = hx
        y = layer(x.to(cuda_device)).detach().cpu().numpy()
        hard = om.hard_mask_from_soft(M.numpy(), "block_sparse16", sparsity_ratio=0.5)
        E = hard if hx == 0.0 else (np.float32(hx) * M.numpy() + np.float32(1.0 - hx) * hard).astype(np.float32)
        ref = x.double().numpy() @ (W.double().numpy() * E).T
        np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-5)


def test_glu_joint_block_flips(cuda_device):
    """The joint update counts flips of block hard types from whole-tensor projections."""
    _, _, sm = _mods()
    from sparseforge_amd.glu import glu_joint_update

    kw = dict(mask_type="structured", hard_mask_type="block_sparse16", mask_metric="hessian_obd",
              sparsity_warmup_steps=0, mask_update_period=1, mask_lr=0.3)
    g = torch.Generator().manual_seed(8)
    mods = []
    for _ in range(2):
        cfg = sm.SparseLinearConfig(**kw)
        cfg.enable_hutchinson = True
        m = sm.SparseLinear(64, 48, sparselinear_config=cfg, bias=False).to(cuda_device)
        with torch.no_grad():
            m.weight.copy_(torch.randn(48, 64, generator=g) * 0.02)
            m.hessian_diag.copy_(torch.rand(48, 64, generator=g) * 1e-3)
            m.mask.copy_(torch.rand(48, 64, generator=g))
        mods.append(m)
    prev = [m.mask.detach().cpu().numpy().copy() for m in mods]
    glu_joint_update(mods[0], mods[1], 3, 0.0)
    for m, p0 in zip(mods, prev):
        now = m.mask.detach().cpu().numpy()
        exp = int(((om.hard_mask_from_soft(p0, "block_sparse16", sparsity_ratio=0.5) > 0.5)
                   ^ (om.hard_mask_from_soft(now, "block_sparse16", sparsity_ratio=0.5) > 0.5)).sum())
        assert int(m.weight.flipped_mask) == exp
