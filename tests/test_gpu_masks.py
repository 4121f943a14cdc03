"""GPU parity of the mask kernels (K6-K8) through the drop-in SparseLinear and the C ABI.

Bar: hard masks and flip counts bit-exact; f32 soft masks / gate targets
within 1e-6 of the reference golden vectors and of the oracle; bf16 within
one bf16 ulp (2^-8 near 1).
"""
import ast

import numpy as np
import pytest
import torch

from conftest import load_golden
from oracle import masks as om
from oracle.numerics import BF16, F32

pytestmark = pytest.mark.gpu


def _sm():
    from sparseforge_amd import sparse_modeling as sm

    return sm


def _K():
    from sparseforge_amd import _lib as L
    from sparseforge_amd import kernels as K

    return L, K


def _hard_parity(got: np.ndarray, ref: np.ndarray, tol: float, gpu_flips: int, ref_flips: int, tag: str) -> int:
    """Hard 2:4 projections of the GPU's soft mask and of the oracle's own soft mask agree except in
    groups whose decision is a genuine near-tie: there the oracle's 2nd and 3rd largest values lie within
    2 * tol (the two soft masks may each sit tol from the true value).  The flip counts differ by at most
    four positions per such group.  Returns the count of such groups (printed)."""
    hg, hr = om.hard_mask_from_soft(got, "nm_2_4"), om.hard_mask_from_soft(ref, "nm_2_4")
    full = (ref.shape[1] // 4) * 4
    diff = (hg[:, :full] != hr[:, :full]).reshape(ref.shape[0], -1, 4).any(-1)
    assert np.array_equal(hg[:, full:], hr[:, full:]), "tail columns are kept by both"
    rows, grps = np.nonzero(diff)
    srt = -np.sort(-ref[:, :full].reshape(ref.shape[0], -1, 4)[rows, grps].astype(np.float64), axis=-1)
    gap = srt[:, 1] - srt[:, 2] if len(rows) else np.zeros(0)
    assert np.all(gap <= 2 * tol), (tag, gap.max(initial=0.0))
    assert abs(gpu_flips - ref_flips) <= 4 * len(rows), (tag, gpu_flips, ref_flips, len(rows))
    print(f"[{tag}] groups {diff.size}, hard decisions differing from the oracle's own mask: {len(rows)} "
          f"(all near-ties, max gap {gap.max(initial=0.0):.2e}); flips gpu {gpu_flips} oracle {ref_flips}")
    return len(rows)


def _tie_heavy(rng, shape):
    vals = np.array([0.0, 1.0, 0.5, 0.25, 0.75, 1.0, 0.0], dtype=np.float32)
    return vals[rng.integers(0, len(vals), size=shape)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("cols", [64, 66, 7, 3, 4096])
def test_nm24_hard_mask_bit_exact(cuda_device, dtype, cols):
    L, K = _K()
    rng = np.random.default_rng(cols)
    rows = 37
    soft = np.where(rng.random((rows, cols)) < 0.5, _tie_heavy(rng, (rows, cols)),
                    rng.random((rows, cols))).astype(np.float32)
    soft = torch.from_numpy(soft).to(dtype)
    ref = om.hard_mask_from_soft(soft.float().numpy(), "nm_2_4")
    got = K.hard_mask(soft.to(cuda_device), L.HARD_NM_TAIL_KEEP, 2, 4)
    assert got.dtype == dtype
    assert np.array_equal(got.float().cpu().numpy(), ref)


@pytest.mark.parametrize("rows, cols", [(4500, 1023), (1100, 4094)])
def test_nm24_hard_mask_multi_stride(cuda_device, rows, cols):
    """More groups than the grid has threads (> 4096 x 256), ragged rows: each thread walks several strides."""
    L, K = _K()
    rng = np.random.default_rng(rows)
    soft = rng.random((rows, cols), dtype=np.float32)
    soft[rng.random((rows, cols)) < 0.3] = 0.5  # ties
    ref = om.hard_mask_from_soft(soft, "nm_2_4")
    got = K.hard_mask(torch.from_numpy(soft).to(cuda_device), L.HARD_NM_TAIL_KEEP, 2, 4)
    assert np.array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("n_keep", [1, 2, 3])
def test_structured_hard_mask_bit_exact(cuda_device, n_keep):
    L, K = _K()
    rng = np.random.default_rng(n_keep)
    soft = torch.from_numpy(_tie_heavy(rng, (129, 256)))
    ref = om.hard_mask_from_soft(soft.numpy(), "structured", N=n_keep, M=4)
    got = K.hard_mask(soft.to(cuda_device), L.HARD_NM_STRICT, n_keep, 4, out_dtype=torch.bfloat16)
    assert np.array_equal(got.float().cpu().numpy(), ref)
    with pytest.raises(ValueError):
        K.hard_mask(soft[:, :6].contiguous().to(cuda_device), L.HARD_NM_STRICT, n_keep, 4)


def test_all_ones_mask_keeps_columns_2_3(cuda_device):
    L, K = _K()
    got = K.hard_mask(torch.ones(5, 16, device=cuda_device), L.HARD_NM_TAIL_KEEP, 2, 4)
    assert (got.cpu() == torch.tensor([0.0, 0, 1, 1]).repeat(5, 4)).all()


def test_empty_mask(cuda_device):
    L, K = _K()
    out = K.hard_mask(torch.empty(0, 8, device=cuda_device), L.HARD_NM_TAIL_KEEP, 2, 4)
    assert out.shape == (0, 8)


def test_flip_count(cuda_device):
    L, K = _K()
    rng = np.random.default_rng(9)
    a = rng.random((64, 130)).astype(np.float32)
    b = a + rng.standard_normal(a.shape).astype(np.float32) * 0.2
    exp = int(((om.hard_mask_from_soft(a, "nm_2_4") > 0.5) ^ (om.hard_mask_from_soft(b, "nm_2_4") > 0.5)).sum())
    cnt = K.hard_flip_count(torch.from_numpy(a).to(cuda_device), torch.from_numpy(b).to(cuda_device),
                            L.HARD_NM_TAIL_KEEP, 2, 4)
    assert int(cnt.item()) == exp


def _dt(name):
    return (BF16, torch.bfloat16) if "bfloat16" in str(name) else (F32, torch.float32)


def _layer_from_golden(r, cfg_kw, tdt, dev, cols=None):
    sm = _sm()
    cfg = sm.SparseLinearConfig(**cfg_kw)
    if cfg_kw.get("mask_metric", "") in ("hessian_ratio", "hessian_obd", "hessian") and r["H"].shape == r["W"].shape:
        cfg.enable_hutchinson = True  # the *_noH_* fixtures keep hessian_diag a placeholder
    W = r["W"]
    layer = sm.SparseLinear(W.shape[1], W.shape[0], sparselinear_config=cfg, bias=False).to(tdt).to(dev)
    layer.weight.mask = layer.mask
    with torch.no_grad():
        layer.weight.copy_(torch.from_numpy(W).to(tdt))
        if not layer._is_placeholder("hessian_diag"):
            layer.hessian_diag.copy_(torch.from_numpy(r["H"]).to(tdt))
    return layer


@pytest.mark.parametrize("case", ["gate_unstr_ratio_f32", "gate_unstr_beta_f32", "gate_unstr_frozen_f32",
                                  "gate_struct_f32", "gate_struct_exact_f32", "gate_unstr_ratio_bf16",
                                  "gate_struct_bf16", "gate_obd_noH_f32", "gate_obd_noH_bf16"])
def test_gate_target_matches_reference(cuda_device, case):
    r = load_golden(case)
    kw = ast.literal_eval(str(r["cfg"]))
    odt, tdt = _dt(r["dtype"])
    layer = _layer_from_golden(r, kw, tdt, cuda_device)
    with torch.no_grad():
        layer.mask.copy_(torch.from_numpy(r["mask"]).to(tdt))
        if not layer._is_placeholder("frozen_mask_flags"):
            layer.frozen_mask_flags.copy_(torch.from_numpy(r["frozen"]).to(tdt))
    idx = torch.from_numpy(r["idx"]).to(cuda_device)
    n = r["W"].size
    G = layer.compute_gate_target(int(r["step"]), sample_idx=idx if idx.numel() < n else None)
    tol = 1e-6 if odt == F32 else 2 ** -8
    np.testing.assert_allclose(G.float().cpu().numpy(), r["G"], rtol=0, atol=tol)


@pytest.mark.parametrize("case", ["update_paper_f32", "update_mid_bin_f32", "update_struct_topn_f32",
                                  "update_freeze_f32", "update_paper_bf16", "update_obd_noH_f32"])
def test_update_mask_matches_reference(cuda_device, case):
    r = load_golden(case)
    kw = ast.literal_eval(str(r["cfg"]))
    odt, tdt = _dt(r["dtype"])
    layer = _layer_from_golden(r, kw, tdt, cuda_device)
    has_frozen = not layer._is_placeholder("frozen_mask_flags")
    with torch.no_grad():
        layer.mask.copy_(torch.from_numpy(r["init_mask"]).to(tdt))
        if has_frozen:
            layer.frozen_mask_flags.copy_(torch.from_numpy(r["init_frozen"]).to(tdt))
    n = r["W"].size
    tol = 1e-6 if odt == F32 else 2 ** -8
    for j, step in enumerate(r["steps"]):
        idx = torch.from_numpy(r[f"idx{j}"]).to(cuda_device)
        layer.update_mask(int(step), lambda_mid=float(r["lam"]), sample_idx=idx if idx.numel() < n else None)
        got = layer.mask.float().cpu().numpy()
        np.testing.assert_allclose(got, r[f"mask{j}"], rtol=0, atol=tol)
        assert int(layer.weight.flipped_mask) == int(r[f"flips{j}"])
        assert layer.hardening_x == float(r[f"hx{j}"])
        if has_frozen:
            assert np.array_equal(layer.frozen_mask_flags.float().cpu().numpy(), r[f"frozen{j}"])
        with torch.no_grad():  # continue from the reference state
            layer.mask.copy_(torch.from_numpy(r[f"mask{j}"]).to(tdt))


@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16])
def test_update_mask_cfg1_shape_matches_oracle(cuda_device, wdt):
    """GPT-2-small MLP shape [3072, 768] with the paper's unstructured + nm_2_4 settings."""
    sm = _sm()
    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio",
                                sparsity_warmup_steps=0, mask_update_period=1, mask_penalty_mode="nm_2_4",
                                mask_penalty_lr=0.1, mask_lr=0.1, temp_init=0.5)
    cfg.enable_hutchinson = True
    g = torch.Generator().manual_seed(0)
    W = (torch.randn(3072, 768, generator=g) * 0.02).to(wdt)
    H = (torch.rand(3072, 768, generator=g) * 1e-3).to(wdt)
    M0 = torch.rand(3072, 768, generator=g).to(wdt)
    layer = sm.SparseLinear(768, 3072, sparselinear_config=cfg, bias=False).to(wdt).to(cuda_device)
    with torch.no_grad():
        layer.weight.copy_(W)
        layer.hessian_diag.copy_(H)
        layer.mask.copy_(M0)
    idx = torch.randint(0, W.numel(), (262144,), generator=g)
    layer.update_mask(7, lambda_mid=0.05, sample_idx=idx.to(cuda_device))
    odt = F32 if wdt == torch.float32 else BF16
    c = om.full_config(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio",
                       sparsity_warmup_steps=0, mask_update_period=1, mask_penalty_mode="nm_2_4",
                       mask_penalty_lr=0.1, mask_lr=0.1, temp_init=0.5)
    new, _, flips, hx = om.layer_update_mask(c, 7, W.float().numpy(), H.float().numpy(), M0.float().numpy(), None,
                                            idx.numpy(), 0.05, odt, odt, odt)
    got = layer.mask.float().cpu().numpy()
    tol = 1e-6 if odt == F32 else 2 ** -8
    np.testing.assert_allclose(got, new, rtol=0, atol=tol)
    # the device projection of the GPU mask is the oracle's projection of it, bit for bit
    hard_gpu = layer._hard_mask_from_soft(layer.mask).float().cpu().numpy()
    assert np.array_equal(hard_gpu, om.hard_mask_from_soft(got, "nm_2_4"))
    # against the oracle's own mask: only genuine near-ties may differ
    _hard_parity(got, new, tol, int(layer.weight.flipped_mask), flips, f"cfg1 {odt}")


def test_update_mask_multi_stride_ragged(cuda_device):
    """[4500, 1023]: 1.15 M groups of 4 with a 3-wide tail per row, more than one grid stride per thread."""
    sm = _sm()
    kw = dict(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio", sparsity_warmup_steps=0,
              mask_update_period=1, mask_penalty_mode="nm_2_4", mask_penalty_lr=0.1, mask_lr=0.1, temp_init=0.5)
    cfg = sm.SparseLinearConfig(**kw)
    cfg.enable_hutchinson = True
    rows, cols = 4500, 1023
    g = torch.Generator().manual_seed(5)
    W = torch.randn(rows, cols, generator=g) * 0.02
    H = torch.rand(rows, cols, generator=g) * 1e-3
    M0 = torch.rand(rows, cols, generator=g)
    layer = sm.SparseLinear(cols, rows, sparselinear_config=cfg, bias=False).to(cuda_device)
    with torch.no_grad():
        layer.weight.copy_(W)
        layer.hessian_diag.copy_(H)
        layer.mask.copy_(M0)
    idx = torch.randint(0, W.numel(), (262144,), generator=g)
    layer.update_mask(3, lambda_mid=0.05, sample_idx=idx.to(cuda_device))
    new, _, flips, _ = om.layer_update_mask(om.full_config(**kw), 3, W.numpy(), H.numpy(), M0.numpy(), None,
                                            idx.numpy(), 0.05)
    got = layer.mask.cpu().numpy()
    np.testing.assert_allclose(got, new, rtol=0, atol=1e-6)
    _hard_parity(got, new, 1e-6, int(layer.weight.flipped_mask), flips, "ragged f32")


def test_tau_quantile_matches_torch(cuda_device):
    sm = _sm()
    cfg = sm.SparseLinearConfig(mask_type="unstructured", tau_sample_size=1000)
    layer = sm.SparseLinear(64, 32, sparselinear_config=cfg, bias=False).to(cuda_device)
    g = torch.Generator().manual_seed(3)
    scores = torch.randn(300, 50, generator=g)
    tau = layer._tau_unstructured(scores.to(cuda_device), 0.37)  # numel 15000 > 1000: sampled on the device
    assert tau.shape == ()
    cfg2 = sm.SparseLinearConfig(mask_type="unstructured", tau_sample_size=10 ** 6)
    layer2 = sm.SparseLinear(64, 32, sparselinear_config=cfg2, bias=False).to(cuda_device)
    for q in (0.0, 0.37, 0.5, 1.0):
        t2 = layer2._tau_unstructured(scores.to(cuda_device), q)
        assert t2.item() == torch.quantile(scores, q).item()


@pytest.mark.parametrize("case", ["gauss", "ties", "nan", "tiny", "ragged"])
def test_tau_quantile_radix_select_large(cuda_device, case):
    """The multi-workgroup radix select equals torch.quantile over 262144 keys (ties, NaN, tiny inputs) and
    over 275561 keys (ragged: the passes' 8-keys-per-round loop plus its remainder loop)."""
    sm = _sm()
    cfg = sm.SparseLinearConfig(mask_type="unstructured", tau_sample_size=10 ** 7)
    layer = sm.SparseLinear(64, 32, sparselinear_config=cfg, bias=False).to(cuda_device)
    g = torch.Generator().manual_seed(17)
    if case == "tiny":
        scores = torch.randn(1, 3, generator=g)
    elif case == "ragged":
        scores = torch.randn(517, 533, generator=g)
    else:
        scores = torch.randn(512, 512, generator=g)
    if case == "ties":
        scores = (scores * 4).round() / 4  # a handful of distinct values, huge tie runs
    if case == "nan":
        scores[7, 9] = float("nan")
    for q in (0.0, 0.25, 0.5, 0.9, 1.0):
        got = layer._tau_unstructured(scores.to(cuda_device), q).item()
        ref = torch.quantile(scores, q).item()
        if case == "nan":
            assert got != got and ref != ref
        else:
            assert got == ref, (case, q, got, ref)


@pytest.mark.parametrize("N,M", [(2, 8), (4, 8), (1, 2)])
def test_structured_group_size_other_than_4_is_rejected(cuda_device, N, M):
    """The device kernels build N:M groups of 4 only (the reference's structured mask takes any M,
    legacy/sparse_modeling.py:720-735, :1164-1185, :1531-1565).  Every entry point that would need another
    group size raises NotImplementedError instead of projecting groups of 4: the hard projection, the
    forward during hardening, the gate target and update_mask."""
    sm = _sm()
    cfg = sm.SparseLinearConfig(mask_type="structured", N=N, M=M, hard_mask_type="match", mask_metric="magnitude",
                                sparsity_warmup_steps=0, mask_update_period=1)
    layer = sm.SparseLinear(64, 16, sparselinear_config=cfg, bias=False).to(cuda_device)
    with torch.no_grad():
        layer.weight.copy_(torch.randn(16, 64) * 0.02)
        layer.mask.copy_(torch.rand(16, 64))
    before = layer.mask.detach().clone()
    with pytest.raises(NotImplementedError):
        layer._hard_mask_from_soft(layer.mask)
    layer.hardening_x = 0.5
    with pytest.raises(NotImplementedError):
        layer(torch.randn(8, 64, device=cuda_device))
    with pytest.raises(NotImplementedError):
        layer.compute_gate_target(1)
    with pytest.raises(NotImplementedError):
        layer.update_mask(1)
    assert torch.equal(layer.mask, before)  # nothing was written
