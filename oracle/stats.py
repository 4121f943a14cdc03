"""Oracle of the mask penalties and statistics (legacy/utils.py).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  numpy restatement of

  mid_penalty        legacy/utils.py:876-938
  sparsity_penalty   legacy/utils.py:942-1025
  nm_2_4_tile_stats  legacy/utils.py:1029-1234
  mask_stats         legacy/utils.py:2069-2280

split the way the device path splits them: `layer_sums` gives the per-layer
sums of one mask (the SF_MSTAT_* row), `hist_counts` the histogram of sampled
values, and the compose_* functions turn per-layer rows into the reference's
scalars.  Mask values are given as float32 arrays holding the stored values
(bf16 masks already rounded); `dt` says which dtype the mask has, because the
reference evaluates m * (1 - m), the entropy clamp and the threshold
comparisons in the mask dtype.
"""
from __future__ import annotations

import math

import numpy as np

from .numerics import rnd

SUM, SUM2, ENTROPY = 0, 1, 2
LT05, LT01, LT001, GT90, GT99, GT05 = 3, 4, 5, 6, 7, 8
SUM_LT05, SUM_GT05, MID, NONFINITE = 9, 10, 11, 12
TOP2, BOT2, TAIL_LT05 = 13, 14, 15
COUNT = 16


def _thr(t: float, dt: str) -> np.float32:
    """A Python float threshold as torch compares it against a tensor of dtype dt."""
    return rnd(np.float32(t), dt).astype(np.float32)


def tile_sums(m2d: np.ndarray):
    """(top2, bot2) f64 sums over the full groups of 4 along each row (:1099-1104, :1175-1185):
    descending sort with NaN first, the first two vs the last two."""
    r, c = m2d.shape
    full = (c // 4) * 4
    if full == 0 or r == 0:
        return 0.0, 0.0
    g = m2d[:, :full].reshape(-1, 4).astype(np.float32)
    key = np.where(np.isnan(g), np.inf, g)  # NaN sorts before every number in a descending sort
    order = np.argsort(-key, axis=1, kind="stable")
    s = np.take_along_axis(g, order, axis=1).astype(np.float64)
    return float(s[:, :2].sum()), float(s[:, 2:].sum())


def layer_sums(m2d: np.ndarray, dt: str, tail_col: int = 0, eps: float = 1e-8) -> np.ndarray:
    """The 16 sums of one mask [rows, cols] (float64)."""
    m = np.asarray(m2d, dtype=np.float32)
    x = m.astype(np.float64).ravel()
    out = np.zeros(COUNT, dtype=np.float64)
    out[SUM] = x.sum()
    out[SUM2] = (x * x).sum()
    # mm = m.clamp(eps, 1 - eps) in the mask dtype, then .double() (:2131-2133)
    lo, hi = np.float32(eps), np.float32(1.0 - eps)
    mf = m.ravel()
    c = np.where(mf < lo, lo, np.where(mf > hi, hi, mf)).astype(np.float32)
    c = rnd(c, dt).astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        ent = -(c * np.log(c)) - ((1.0 - c) * np.log(1.0 - c))
    out[ENTROPY] = ent.sum()
    with np.errstate(invalid="ignore"):
        out[LT05] = np.count_nonzero(mf < np.float32(0.5))
        out[LT01] = np.count_nonzero(mf < _thr(0.1, dt))
        out[LT001] = np.count_nonzero(mf < _thr(0.01, dt))
        out[GT90] = np.count_nonzero(mf > _thr(0.9, dt))
        out[GT99] = np.count_nonzero(mf > _thr(0.99, dt))
        out[GT05] = np.count_nonzero(mf > np.float32(0.5))
        out[SUM_LT05] = x[mf < np.float32(0.5)].sum()
        out[SUM_GT05] = x[mf > np.float32(0.5)].sum()
    # local_penalty = (m * (1 - m)).sum(): 1 - m and the product in the mask dtype (:911)
    om = rnd(np.float32(1.0) - mf, dt).astype(np.float32)
    out[MID] = rnd((mf * om).astype(np.float32), dt).astype(np.float64).sum()
    out[NONFINITE] = np.count_nonzero(~np.isfinite(mf))
    out[TOP2], out[BOT2] = tile_sums(m)
    if m.ndim == 2 and tail_col < m.shape[1]:
        with np.errstate(invalid="ignore"):
            out[TAIL_LT05] = np.count_nonzero(m[:, max(tail_col, 0):] < np.float32(0.5))
    return out


def hist_counts(values: np.ndarray, bins: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    """torch.histc's device binning of float32 values: b = (int)((x - lo) * bins / (hi - lo)) in
    float32, b == bins -> bins - 1; NaN and values outside [lo, hi] are not counted."""
    x = np.asarray(values, dtype=np.float32)
    with np.errstate(invalid="ignore"):
        ok = (x >= np.float32(lo)) & (x <= np.float32(hi))
    x = x[ok]
    b = ((x - np.float32(lo)) * np.float32(bins) / (np.float32(hi) - np.float32(lo))).astype(np.float32)
    b = np.minimum(np.trunc(b).astype(np.int64), bins - 1)
    return np.bincount(b, minlength=bins).astype(np.int64)


def round_sum(x: float, dt: str) -> float:
    """A float64 sum as torch's .sum() over a dt tensor returns it (result in the tensor dtype)."""
    return float(rnd(np.float32(x), dt))


def compose_mid_penalty(rows, dts, numels, lambda_mid: float) -> float:
    """:893-938"""
    if lambda_mid <= 0:
        return 0.0
    pen = cnt = 0.0
    for r, dt, n in zip(rows, dts, numels):
        if r[NONFINITE] > 0:
            continue
        pen += round_sum(r[MID], dt)
        cnt += float(n)
    if cnt <= 0:
        return 0.0
    res = lambda_mid * (pen / cnt)
    return 0.0 if not math.isfinite(res) else float(np.float32(res))


def compose_sparsity(layers, target_sparsity: float, alpha: float):
    """:953-1025.  layers: (row, kind, shape, N, M) with kind 'structured' or other."""
    cnt = tot = 0.0
    for r, kind, shape, N, M in layers:
        if kind == "structured" and len(shape) == 2 and (shape[1] // M) * M > 0:
            out_dim, in_dim = shape
            in_full = (in_dim // M) * M
            tot += float(out_dim * in_full)
            cnt += float(out_dim * (in_full // M) * (M - N))
            if in_full < in_dim:
                tot += float(out_dim * (in_dim - in_full))
                cnt += r[TAIL_LT05]
        else:
            tot += float(np.prod(shape))
            cnt += r[LT05]
    cur = 0.0 if tot <= 0 else cnt / tot
    pen = float(alpha * (cur - target_sparsity) ** 2) if alpha != 0.0 else 0.0
    return pen, cur


def compose_tile_stats(rows, tiles):
    """:1187-1234; the per-layer sums are float32 in the reference."""
    total = float(sum(tiles))
    if total <= 0:
        return {"top2_avg": 0.0, "bot2_avg": 0.0, "top2_gap": 0.0, "bot2_gap": 0.0, "total_gap": 0.0}
    top = sum(float(np.float32(r[TOP2])) for r in rows)
    bot = sum(float(np.float32(r[BOT2])) for r in rows)
    t2, b2 = top / (total * 2), bot / (total * 2)
    return {"top2_avg": t2, "bot2_avg": b2, "top2_gap": 1.0 - t2, "bot2_gap": b2, "total_gap": (1.0 - t2) + b2}


def quantile_from_hist(hist: np.ndarray, q: float, mean: float) -> float:
    """_q_from_hist (:2232-2243): first bin whose CDF >= q (q compared as float32), bin centre."""
    h = np.asarray(hist, dtype=np.float64)
    bins = h.size
    if h.sum() <= 0:
        return mean
    cdf = np.cumsum(h) / (h.sum() + 1e-12)
    i = int(np.searchsorted(cdf, np.float64(np.float32(q)), side="left"))
    return float((max(0, min(bins - 1, i)) + 0.5) / bins)


def compose_mask_stats(rows, numels, hist, blocks=None):
    """:2188-2280.  blocks: list of per-layer block-mean vectors (block_sparse layers)."""
    tot = float(sum(numels))
    if tot <= 0:
        return {"mask_mean": 1.0, "mask_std": 0.0, "mask_entropy": 0.0, "mask_hard_sparsity@0.5": 0.0,
                "mask_frac_lt_0.1": 0.0, "mask_frac_lt_0.01": 0.0, "mask_p10": 1.0, "mask_p50": 1.0,
                "mask_p90": 1.0}
    s = np.sum(np.asarray(rows, dtype=np.float64), axis=0)
    mean = s[SUM] / tot
    std = math.sqrt(max(s[SUM2] / tot - mean * mean, 0.0))
    res = {
        "mask_mean": mean, "mask_std": std, "mask_entropy": s[ENTROPY] / tot,
        "mask_hard_sparsity@0.5": s[LT05] / tot, "mask_frac_lt_0.1": s[LT01] / tot,
        "mask_frac_lt_0.01": s[LT001] / tot, "mask_frac_gt_0.9": s[GT90] / tot,
        "mask_frac_gt_0.99": s[GT99] / tot, "mask_frac_gt_0.5": s[GT05] / tot,
        "mask_mean_lt_0.5": s[SUM_LT05] / s[LT05] if s[LT05] > 0 else 0.0,
        "mask_mean_gt_0.5": s[SUM_GT05] / s[GT05] if s[GT05] > 0 else 0.0,
        "mask_p10": quantile_from_hist(hist, 0.10, mean),
        "mask_p50": quantile_from_hist(hist, 0.50, mean),
        "mask_p90": quantile_from_hist(hist, 0.90, mean),
    }
    if blocks:
        nb = lo_s = lo_c = up_s = up_c = 0.0
        for v in blocks:
            v = np.sort(np.asarray(v, dtype=np.float32))
            n = v.size
            nb += n
            half = n // 2
            if half > 0:
                lo_s += v[:half].astype(np.float64).sum()
                lo_c += half
                up_s += v[half:].astype(np.float64).sum()
                up_c += n - half
        if nb > 0:
            lo_m = lo_s / lo_c if lo_c > 0 else 0.0
            up_m = up_s / up_c if up_c > 0 else 0.0
            res.update({"blk_lower_half_mean": lo_m, "blk_upper_half_mean": up_m, "blk_total_blocks": nb,
                        "blk_separation": up_m - lo_m})
    return res
