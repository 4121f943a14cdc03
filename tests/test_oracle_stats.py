"""Pins the penalty / mask-statistics oracle (oracle/stats.py) — CPU only.

* mid_penalty, sparsity_penalty, nm_2_4_tile_stats and mask_stats composed
  from the oracle's per-layer sums against golden vectors the reference code
  wrote (tests/golden/make_reference_golden.py, group `stats`): f32 and bf16
  masks, ragged rows, values on and next to every threshold, block_sparse
  layers, a layer holding NaN and an exact 1 (entropy NaN);
* the group-of-4 sort against Python's sorted() with NaN first;
* the histogram binning against torch.histc away from bin edges;
* closed forms: constant masks.
"""
import math

import numpy as np
import pytest
import torch

from conftest import load_golden
from oracle import masks as om
from oracle import stats as ost

CASES = ["stats_f32", "stats_bf16", "stats_nan_f32"]


def _layers(g):
    out = []
    for i in range(int(g["n_layers"])):
        m = g[f"mask{i}"]
        out.append((m, str(g[f"mask_type{i}"]), str(g[f"hard_type{i}"])))
    return out


def _rows(g, eps=1e-8):
    dt = str(g["dtype"])
    rows = []
    for m, mt, _ in _layers(g):
        tail = (m.shape[1] // 4) * 4 if mt == "structured" else 0
        rows.append(ost.layer_sums(m, dt, tail, eps))
    return rows


def _close(a, b, rtol):
    if isinstance(b, float) and math.isnan(b):
        return math.isnan(a)
    return a == pytest.approx(b, rel=rtol, abs=1e-12)


@pytest.mark.parametrize("name", CASES)
def test_mid_penalty_golden(name):
    g = load_golden(name)
    ls = _layers(g)
    got = ost.compose_mid_penalty(_rows(g), [str(g["dtype"])] * len(ls), [m.size for m, _, _ in ls], 0.7)
    assert _close(got, float(g["mid"]), 1e-6)


@pytest.mark.parametrize("name", CASES)
def test_sparsity_penalty_golden(name):
    g = load_golden(name)
    layers = [(r, mt, m.shape, 2, 4) for r, (m, mt, _) in zip(_rows(g), _layers(g))]
    pen, cur = ost.compose_sparsity(layers, 0.4, 2.0)
    assert cur == float(g["sp_cur"])
    assert _close(pen, float(g["sp_pen"]), 1e-6)


@pytest.mark.parametrize("name", CASES)
def test_tile_stats_golden(name):
    g = load_golden(name)
    ls = _layers(g)
    got = ost.compose_tile_stats(_rows(g), [m.shape[0] * (m.shape[1] // 4) for m, _, _ in ls])
    for k, v in zip(g["tile_keys"], g["tile_vals"]):
        assert _close(got[str(k)], float(v), 1e-6), k


@pytest.mark.parametrize("name", CASES)
def test_mask_stats_golden(name):
    g = load_golden(name)
    ls = _layers(g)
    hist = np.zeros(100, dtype=np.int64)
    blocks = []
    for i, (m, _, ht) in enumerate(ls):
        hist += ost.hist_counts(m.ravel()[g[f"idx{i}"]], 100)
        if ht in ("block_sparse16", "block_sparse32"):
            bs = 16 if ht == "block_sparse16" else 32
            if m.shape[0] >= bs and m.shape[1] >= bs:
                blocks.append(om.block_mean(m, bs).ravel())
    got = ost.compose_mask_stats(_rows(g), [m.size for m, _, _ in ls], hist, blocks)
    want = {str(k): float(v) for k, v in zip(g["ms_keys"], g["ms_vals"])}
    assert set(got) == set(want)
    for k, v in want.items():
        if k == "blk_separation":  # a difference of two f32 means: absolute tolerance of a few f32 ulp
            assert abs(float(got[k]) - v) < 1e-6, (k, got[k], v)
        else:
            assert _close(float(got[k]), v, 1e-6), (k, got[k], v)


def test_tile_sort_nan_first_bruteforce():
    rng = np.random.default_rng(3)
    vals = np.array([0.0, -0.0, 0.25, 0.5, 1.0, np.nan, -1.0], dtype=np.float32)
    m = vals[rng.integers(0, len(vals), size=(40, 23))]
    top = bot = 0.0
    for row in m:
        for c in range(0, 20, 4):
            grp = sorted(row[c:c + 4].tolist(), key=lambda v: (not math.isnan(v), -v if not math.isnan(v) else 0))
            top += grp[0] + grp[1]
            bot += grp[2] + grp[3]
    t, b = ost.tile_sums(m)
    assert _close(t, top, 1e-12) and _close(b, bot, 1e-12)


def test_hist_binning_matches_torch_histc_off_edges():
    rng = np.random.default_rng(5)
    x = rng.uniform(-0.2, 1.2, 200000).astype(np.float32)
    x = x[np.abs(x * 100 - np.round(x * 100)) > 1e-3]  # no value within float rounding of a bin edge
    want = torch.histc(torch.from_numpy(x), bins=100, min=0.0, max=1.0).numpy().astype(np.int64)
    assert (ost.hist_counts(x, 100) == want).all()
    # both ends of the range are counted, the top end in the last bin; NaN is not counted
    h = ost.hist_counts(np.array([0.0, 1.0, np.nan, -1e-7, 1.0000001], np.float32), 100)
    assert h[0] == 1 and h[99] == 1 and h.sum() == 2


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_constant_half_mask_closed_form(dt):
    m = np.full((8, 12), 0.5, np.float32)
    r = ost.layer_sums(m, dt)
    assert r[ost.MID] == 0.25 * m.size
    assert r[ost.TOP2] == r[ost.BOT2] == 0.5 * 2 * (m.size // 4)
    assert r[ost.LT05] == r[ost.GT05] == 0
    assert r[ost.ENTROPY] == pytest.approx(math.log(2.0) * m.size, rel=1e-12)
    s = ost.compose_mask_stats([r], [m.size], ost.hist_counts(m.ravel(), 100))
    assert s["mask_mean"] == 0.5 and s["mask_std"] == 0.0 and s["mask_p50"] == 0.505
    assert ost.compose_mid_penalty([r], [dt], [m.size], 2.0) == pytest.approx(0.5)


def test_all_ones_mask_closed_form():
    m = np.ones((4, 8), np.float32)
    r = ost.layer_sums(m, "f32")
    assert math.isnan(r[ost.ENTROPY])  # clamp(1 - 1e-8) is 1.0 in float32: (1 - 1) * log(0)
    assert ost.compose_mid_penalty([r], ["f32"], [m.size], 1.0) == 0.0
    assert ost.compose_sparsity([(r, "structured", m.shape, 2, 4)], 0.5, 1.0) == (0.0, 0.5)
    assert ost.compose_sparsity([(r, "unstructured", m.shape, 2, 4)], 0.5, 1.0) == (0.25, 0.0)
