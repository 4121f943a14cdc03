"""GPU parity of the mask penalties and statistics (sf_mask_stats, sf_mask_hist,
sf_keep_split_sum; utils.mid_penalty / sparsity_penalty / nm_2_4_tile_stats / mask_stats).

Bar: counts bit-exact against the oracle; f64 sums within 1e-12 relative (the
summation order differs), the entropy sum (f32 terms) within 1e-6, the NaN / inf cases NaN where the oracle is; the
model-level scalars within 1e-6 of the reference's own outputs
(tests/golden/ref_stats_*), whose histogram quantiles are replayed from the
same torch.randint draws on the GPU.
"""
import math

import numpy as np
import pytest
import torch

from conftest import load_golden
from oracle import stats as ost

pytestmark = pytest.mark.gpu


def _mods():
    from sparseforge_amd import _lib as L
    from sparseforge_amd import kernels as K
    from sparseforge_amd import sparse_modeling as sm
    from sparseforge_amd import utils as U

    return L, K, sm, U


def _dev_rows(mask: torch.Tensor, tail=0, eps=1e-8):
    L, K, _, _ = _mods()
    out = torch.empty(L.MSTAT_COUNT, dtype=torch.float64, device=mask.device)
    K.mask_stats(mask, out, tail, eps)
    return out.cpu().numpy()


def _check_row(got, want):
    for k in range(ost.COUNT):
        if math.isnan(want[k]):
            assert math.isnan(got[k]), k
        elif k in (ost.LT05, ost.LT01, ost.LT001, ost.GT90, ost.GT99, ost.GT05, ost.NONFINITE, ost.TAIL_LT05):
            assert got[k] == want[k], (k, got[k], want[k])
        elif k == ost.ENTROPY:  # f32 terms on the device, f64 logs in the reference and the oracle
            assert got[k] == pytest.approx(want[k], rel=1e-6, abs=1e-9), (k, got[k], want[k])
        else:
            assert got[k] == pytest.approx(want[k], rel=1e-12, abs=1e-9), (k, got[k], want[k])


SHAPES = [(1, 1), (3, 5), (7, 4), (33, 130), (64, 257), (256, 1024), (1024, 4100)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layer_sums_match_oracle(cuda_device, shape, dtype):
    print(f"[stats] layer sums {shape} {dtype}", flush=True)
    g = torch.Generator().manual_seed(shape[0] * 1000 + shape[1])
    m = torch.rand(shape, generator=g)
    specials = torch.tensor([0.0, 1e-9, 0.01, 0.1, 0.5, 0.9, 0.99, 0.999, -0.5])
    n = min(m.numel(), specials.numel())
    m.view(-1)[:n] = specials[:n]
    m = m.to(dtype)
    dt = "bf16" if dtype == torch.bfloat16 else "f32"
    tail = (shape[1] // 4) * 4
    got = _dev_rows(m.to(cuda_device), tail)
    want = ost.layer_sums(m.float().numpy(), dt, tail)
    _check_row(got, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_entropy_of_nearly_hard_masks(cuda_device, dtype):
    """Masks within 2e-3 (f32) / 2e-2 (bf16) of 0 and 1, as late in hardening, where fl(1 - c) drops
    the low bits of a small c and both entropy terms are small: the entropy sum within 1e-6 of the
    oracle's f64 logs, and every other slot to its usual bar."""
    g = torch.Generator().manual_seed(17)
    r = torch.rand(512, 1024, generator=g, dtype=torch.float64)
    span, gap = (2e-3, 2e-6) if dtype == torch.float32 else (2e-2, 2.0 ** -8)  # gap: below 1 in the dtype
    near = torch.where(r < 0.5, r * span + 1e-9, 1 - gap - (r - 0.5) * span).float()
    near.view(-1)[:4] = torch.tensor([3e-8, 1e-7, 2.0 ** -24, 1 - gap])
    m = near.to(dtype)
    assert not bool((m == 1).any())
    dt = "bf16" if dtype == torch.bfloat16 else "f32"
    got = _dev_rows(m.to(cuda_device), 1024)
    want = ost.layer_sums(m.float().numpy(), dt, 1024)
    assert want[ost.ENTROPY] > 0
    _check_row(got, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layer_sums_nan_inf_and_ones(cuda_device, dtype):
    m = torch.rand(16, 22)
    m[0, 1], m[2, 5], m[3, 3], m[5, 21] = float("nan"), float("inf"), 1.0, -float("inf")
    m = m.to(dtype)
    dt = "bf16" if dtype == torch.bfloat16 else "f32"
    got = _dev_rows(m.to(cuda_device), 20)
    want = ost.layer_sums(m.float().numpy(), dt, 20)
    assert want[ost.NONFINITE] == 3 and math.isnan(want[ost.ENTROPY])
    _check_row(got, want)


def test_layer_sums_unaligned_view_and_1d(cuda_device):
    base = torch.rand(4 * 1000 + 1, device=cuda_device)
    m1 = base[1:].view(40, 100)  # 4-byte offset: the scalar path
    _check_row(_dev_rows(m1.contiguous() if not m1.is_contiguous() else m1),
               ost.layer_sums(m1.cpu().numpy(), "f32"))
    flat = torch.rand(1003, device=cuda_device)
    _check_row(_dev_rows(flat), ost.layer_sums(flat.cpu().numpy()[None, :], "f32"))


def test_mask_stats_repeatable(cuda_device):
    m = torch.rand(2048, 2048, device=cuda_device)
    a, b = _dev_rows(m), _dev_rows(m)
    assert (a == b).all()


def test_hist_matches_oracle(cuda_device):
    _, K, _, _ = _mods()
    m = torch.rand(300, 77) * 1.2 - 0.1
    m.view(-1)[:6] = torch.tensor([0.0, 1.0, float("nan"), 0.5, 0.25, 0.99])
    idx = torch.randint(0, m.numel(), (5000,))
    idx[:3] = torch.tensor([0, 1, 2])
    hist = torch.zeros(100, dtype=torch.int64, device=cuda_device)
    for dtype in (torch.float32, torch.bfloat16):
        md = m.to(dtype)
        K.mask_hist(md.to(cuda_device), idx.to(cuda_device), 100, 0.0, 1.0, hist)
    want = sum(ost.hist_counts(m.to(d).float().numpy().ravel()[idx.numpy()], 100)
               for d in (torch.float32, torch.bfloat16))
    assert (hist.cpu().numpy() == want).all()


def test_hist_skips_out_of_range_indices(cuda_device):
    _, K, _, _ = _mods()
    m = torch.full((10,), 0.55, device=cuda_device)
    idx = torch.tensor([-1, 0, 9, 10, 1 << 40], dtype=torch.int64, device=cuda_device)
    hist = torch.zeros(100, dtype=torch.int64, device=cuda_device)
    K.mask_hist(m, idx, 100, 0.0, 1.0, hist)
    assert int(hist.sum()) == 2 and int(hist[55]) == 2


def test_keep_split_sum(cuda_device):
    _, K, _, _ = _mods()
    v = torch.rand(5000, device=cuda_device)
    keep = K.topk_keep(v, 5000 - 2500)
    s = K.keep_split_sum(v, keep).cpu().numpy()
    vs = np.sort(v.cpu().numpy())
    assert s[1] == pytest.approx(vs[:2500].astype(np.float64).sum(), rel=1e-12)
    assert s[0] == pytest.approx(vs[2500:].astype(np.float64).sum(), rel=1e-12)


def _model_from_golden(g, dev):
    _, _, sm, _ = _mods()
    dtype = torch.bfloat16 if str(g["dtype"]) == "bf16" else torch.float32
    model = torch.nn.Module()
    for i in range(int(g["n_layers"])):
        m = torch.from_numpy(g[f"mask{i}"])
        cfg = sm.SparseLinearConfig(mask_type=str(g[f"mask_type{i}"]), hard_mask_type=str(g[f"hard_type{i}"]))
        layer = sm.SparseLinear(m.shape[1], m.shape[0], sparselinear_config=cfg, bias=False).to(dtype).to(dev)
        with torch.no_grad():
            layer.mask.copy_(m.to(dtype))
        model.add_module(f"l{i}", layer)
    return model


def _close(a, b, rtol=1e-6):
    if math.isnan(b):
        return math.isnan(a)
    return a == pytest.approx(b, rel=rtol, abs=1e-12)


@pytest.mark.parametrize("name", ["stats_f32", "stats_bf16", "stats_nan_f32"])
def test_model_level_functions_match_reference(cuda_device, name):
    print(f"[stats] model-level {name}", flush=True)
    _, _, _, U = _mods()
    g = load_golden(name)
    model = _model_from_golden(g, cuda_device)
    assert _close(float(U.mid_penalty(model, 0.7)), float(g["mid"]))
    pen, cur = U.sparsity_penalty(model, 0.4, 2.0)
    assert cur == float(g["sp_cur"]) and _close(float(pen), float(g["sp_pen"]))
    ts = U.nm_2_4_tile_stats(model)
    for k, v in zip(g["tile_keys"], g["tile_vals"]):
        assert _close(ts[str(k)], float(v)), k
    # mask_stats draws its samples with torch.randint on the GPU: replay the draws for the oracle
    sample, seed = int(g["sample"]), 777
    torch.manual_seed(seed)
    ms = U.mask_stats(model, bins=100, sample_per_layer=sample)
    torch.manual_seed(seed)
    hist = np.zeros(100, dtype=np.int64)
    for i in range(int(g["n_layers"])):
        m = g[f"mask{i}"]
        idx = torch.randint(0, m.size, (min(m.size, sample),), device=cuda_device).cpu().numpy()
        hist += ost.hist_counts(m.ravel()[idx], 100)
    want = {str(k): float(v) for k, v in zip(g["ms_keys"], g["ms_vals"])}
    mean = want["mask_mean"]
    for q, k in ((0.10, "mask_p10"), (0.50, "mask_p50"), (0.90, "mask_p90")):
        want[k] = ost.quantile_from_hist(hist, q, mean)
    assert set(ms) == set(want)
    for k, v in want.items():
        if k == "blk_separation":
            assert abs(ms[k] - v) < 1e-6, (k, ms[k], v)
        else:
            assert _close(float(ms[k]), v), (k, ms[k], v)


def test_mid_penalty_zero_lambda_and_empty(cuda_device):
    _, _, sm, U = _mods()
    model = torch.nn.Module()
    model.add_module("l0", sm.SparseLinear(8, 4, sparselinear_config=sm.SparseLinearConfig(), bias=False)
                     .to(cuda_device))
    assert float(U.mid_penalty(model, 0.0)) == 0.0
    with torch.no_grad():
        model.l0.mask.fill_(0.5)
    assert float(U.mid_penalty(model, 2.0)) == pytest.approx(0.5)
    empty = torch.nn.Module()
    assert U.mask_stats(empty)["mask_mean"] == 1.0
    assert U.nm_2_4_tile_stats(empty)["top2_avg"] == 0.0


def test_harden_fraction_matches_reference(cuda_device):
    _, _, sm, U = _mods()
    g = load_golden("harden_f32")
    model = torch.nn.Module()
    for li in range(2):
        m = torch.from_numpy(g[f"mask_in{li}"])
        cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="nm_2_4", freeze_low=0.05,
                                    freeze_high=0.95)
        layer = sm.SparseLinear(m.shape[1], m.shape[0], sparselinear_config=cfg, bias=False).to(cuda_device)
        with torch.no_grad():
            layer.mask.copy_(m)
            layer.frozen_mask_flags.copy_(torch.from_numpy(g[f"frozen_in{li}"]))
        model.add_module(f"l{li}", layer)
    assert U.harden_fraction(model, 0.2, 0.4, 0.6) == int(g["count"])
    for li, layer in enumerate(model.children()):
        assert (layer.mask.detach().cpu().numpy() == g[f"mask_out{li}"]).all()
        assert (layer.frozen_mask_flags.detach().float().cpu().numpy() == g[f"frozen_out{li}"]).all()


def test_shared_mask_rows_reuses_and_invalidates(cuda_device):
    """Inside utils.shared_mask_rows a repeated request for the same masks returns the first rows; an in-place
    change of a mask (its version moves) makes the next request compute them again."""
    _, _, _, U = _mods()
    g = torch.Generator(device=cuda_device).manual_seed(4)
    masks = [torch.rand(64, 96, generator=g, device=cuda_device) for _ in range(2)]
    with U.shared_mask_rows():
        r1 = U._mask_rows(masks)
        assert U._mask_rows(masks) is r1
        masks[0].mul_(0.5)
        r3 = U._mask_rows(masks)
        assert r3 is not r1
        assert not torch.equal(r3[0], r1[0]) and torch.equal(r3[1], r1[1])
    r4 = U._mask_rows(masks)
    assert r4 is not r3 and torch.equal(r4, r3)
