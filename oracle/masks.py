"""Oracle of the mask path: hard projection, scores, gate target and update_mask.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  numpy float32 arithmetic
in the reference's op order; bf16 tensors are emulated by rounding each op's
result (numerics.rnd).  Reference: legacy/sparse_modeling.py of
liuhanzuo/SparseForge.
"""
from __future__ import annotations

import json
import math
import os

import numpy as np

from .numerics import BF16, F32, ordered_keys, promote, rnd, round_bf16, sigmoid_f32
from .select import topk_keep as select_topk_keep

_TIES_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tests", "golden",
                          "topk_ties_m4.json")
_TIES = None


def _ties() -> np.ndarray:
    """[3, 256] keep-bitmask tables of torch.topk(k=1..3) over groups of 4 (fixture data)."""
    global _TIES
    if _TIES is None:
        with open(_TIES_PATH) as f:
            d = json.load(f)
        t = np.zeros((3, 256), dtype=np.uint8)
        for k in range(1, 4):
            for key, row in d["tables"][str(k)].items():
                t[k - 1, int(key)] = row["keep"]
        _TIES = t
    return _TIES


def group_keys(g: np.ndarray) -> np.ndarray:
    """Weak-ordering key of each group of 4: sum_i #{j: v_j < v_i} << 2i."""
    k = ordered_keys(g)
    lt = (k[..., None, :] < k[..., :, None]).sum(-1)  # lt[..., i] = #{j : k_j < k_i}
    return (lt << (2 * np.arange(4))).sum(-1)


def topk_keep(groups: np.ndarray, k: int) -> np.ndarray:
    """Boolean [..., 4]: members torch.topk(groups, k, dim=-1) selects (CPU tie order)."""
    assert groups.shape[-1] == 4 and 1 <= k <= 3
    bits = _ties()[k - 1][group_keys(groups)]
    return ((bits[..., None] >> np.arange(4)) & 1).astype(bool)


def kth_largest(groups: np.ndarray, k: int) -> np.ndarray:
    """topk(k).values[..., -1] with NaN largest."""
    keys = ordered_keys(groups)
    order = np.argsort(-keys.astype(np.int64), axis=-1, kind="stable")
    return np.take_along_axis(groups, order[..., k - 1:k], axis=-1)[..., 0]


# ---------------------------------------------------------------------------
# bs x bs blocks of the fully covered core [:rows // bs * bs, :cols // bs * bs]
# ---------------------------------------------------------------------------
BLOCK_SPARSE = ("block_sparse16", "block_sparse32")
BLOCK_SIZE = {"block16": 16, "block_sparse16": 16, "block_sparse32": 32}


def block_core(shape, bs: int):
    rows, cols = shape
    return (rows // bs) * bs, (cols // bs) * bs


def block_tiles(x: np.ndarray, bs: int) -> np.ndarray:
    """[ob, ib, bs*bs]: each tile's elements in row-major order (the reference's permute(0, 2, 1, 3))."""
    of, inf = block_core(x.shape, bs)
    ob, ib = of // bs, inf // bs
    return np.asarray(x, dtype=np.float32)[:of, :inf].reshape(ob, bs, ib, bs).transpose(0, 2, 1, 3).reshape(
        ob, ib, bs * bs)


def block_expand(b: np.ndarray, bs: int) -> np.ndarray:
    """[ob, ib] -> [ob*bs, ib*bs], every element of a block set to the block's value."""
    return np.repeat(np.repeat(np.asarray(b, dtype=np.float32), bs, axis=0), bs, axis=1)


def block_mean(x: np.ndarray, bs: int) -> np.ndarray:
    """tiles.mean() in float32 per block ([ob, ib]).  The mean is taken in float64 and rounded
    once; torch accumulates in float32, so the two may differ in the last bits (both are exact
    for blocks whose elements are all equal)."""
    return block_tiles(x, bs).astype(np.float64).mean(-1).astype(np.float32)


def block_rms(x: np.ndarray, bs: int) -> np.ndarray:
    """(tiles ** 2).mean().sqrt() per block: square in f32, mean as in block_mean, sqrt in f32."""
    t = block_tiles(x, bs)
    sq = (t * t).astype(np.float32)
    return np.sqrt(sq.astype(np.float64).mean(-1).astype(np.float32)).astype(np.float32)


def topk_keep_desc(v: np.ndarray, k: int) -> np.ndarray:
    """Boolean mask of the entries torch.topk(v, k, dim=-1) keeps (CPU kernel, NaN largest), per row
    of the last axis, equal values included exactly as torch's selection leaves them (oracle.select)."""
    return select_topk_keep(v, k)


def keep_count(frac_kept: float, total: int) -> int:
    """int(round((1 - sr) * total)) clipped to [0, total] (Python round: half to even)."""
    return max(0, min(total, int(round(frac_kept * total))))


def block_hard(soft: np.ndarray, hard_type: str, sparsity_ratio: float) -> np.ndarray:
    """block16 (:537-575): top-k elements inside each 16x16 tile, k = round((1 - sr) 256);
    block_sparse16 / 32 (:607-718): the round((1 - sr) nblocks) blocks of largest RMS kept whole.
    Elements outside the fully covered core stay 1."""
    bs = BLOCK_SIZE[hard_type]
    hard = np.ones_like(soft, dtype=np.float32)
    of, inf = block_core(soft.shape, bs)
    if of == 0 or inf == 0:
        return hard
    ob, ib = of // bs, inf // bs
    if hard_type == "block16":
        k = keep_count(1.0 - sparsity_ratio, bs * bs)
        keep = topk_keep_desc(block_tiles(soft, bs), k).astype(np.float32)
        hard[:of, :inf] = keep.reshape(ob, ib, bs, bs).transpose(0, 2, 1, 3).reshape(of, inf)
    else:
        k = keep_count(1.0 - sparsity_ratio, ob * ib)
        keep = topk_keep_desc(block_rms(soft, bs).ravel(), k).reshape(ob, ib)
        hard[:of, :inf] = block_expand(keep, bs)
    return hard


def blockify(t: np.ndarray, hard_type: str, dt: str) -> np.ndarray:
    """_blockify_tensor (:460-507): block mean over the core for block_sparse16/32, cast to dt."""
    if hard_type not in BLOCK_SPARSE or np.asarray(t).ndim != 2:
        return t
    bs = BLOCK_SIZE[hard_type]
    of, inf = block_core(t.shape, bs)
    if of == 0 or inf == 0:
        return t
    out = np.asarray(t, dtype=np.float32).copy()
    out[:of, :inf] = rnd(block_expand(block_mean(t, bs), bs), dt)
    return out


# ---------------------------------------------------------------------------
# _hard_mask_from_soft (sparse_modeling.py:510-735)
# ---------------------------------------------------------------------------
def hard_mask_from_soft(soft: np.ndarray, hard_type: str, N: int = 2, M: int = 4,
                        sparsity_ratio: float = 0.5) -> np.ndarray:
    soft = np.asarray(soft, dtype=np.float32)
    if hard_type == "none":  # :523-524
        return np.ones_like(soft)
    if hard_type == "unstructured" or soft.ndim == 1:  # :526-531
        return (soft > 0.5).astype(np.float32)
    if hard_type == "nm_2_4":  # :578-603, N=2 M=4 fixed, tail columns kept
        rows, cols = soft.shape
        full = (cols // 4) * 4
        hard = np.ones_like(soft)
        if full:
            g = soft[:, :full].reshape(rows, full // 4, 4)
            hard[:, :full] = topk_keep(g, 2).reshape(rows, full).astype(np.float32)
        return hard
    if hard_type == "structured":  # :720-735
        rows, cols = soft.shape
        if cols % M != 0:
            raise ValueError(f"in_features ({cols}) must be divisible by M ({M}).")
        assert M == 4
        g = soft.reshape(rows, cols // M, M)
        return topk_keep(g, N).reshape(rows, cols).astype(np.float32)
    if hard_type in BLOCK_SIZE:
        return block_hard(soft, hard_type, sparsity_ratio)
    raise ValueError(f"Invalid hard mask_type: {hard_type}")


# ---------------------------------------------------------------------------
# scores and z-normalisation (sparse_modeling.py:1041-1088)
# ---------------------------------------------------------------------------
def score_dtype(metric: str, w_dt: str, h_dt: str, aux_dt: str = F32) -> str:
    if metric in ("hessian_obd", "hessian_ratio"):
        return promote(w_dt, h_dt)
    if metric == "hessian":
        return h_dt
    if metric in ("wanda", "movement"):
        return promote(w_dt, aux_dt)
    return w_dt


def scores(W, H, aux, metric: str, w_dt: str = F32, h_dt: str = F32, aux_dt: str = F32, eps: float = 1e-8,
           temperature: float = 1.0) -> np.ndarray:
    W = np.asarray(W, dtype=np.float32)
    e = np.float32(eps)
    if metric == "magnitude":
        return np.abs(W)
    if metric == "hessian_obd":
        H = np.asarray(H, dtype=np.float32)
        return rnd(rnd(H + e, h_dt) * rnd(W * W, w_dt), promote(h_dt, w_dt))
    if metric == "hessian_ratio":
        H = np.asarray(H, dtype=np.float32)
        return rnd(np.abs(W) / rnd(np.sqrt(rnd(H + e, h_dt)), h_dt), promote(h_dt, w_dt))
    if metric == "hessian":
        return np.asarray(H, dtype=np.float32)
    if metric == "weight_squared":  # hessian_obd without a Hessian (:1053-1055)
        return rnd(W * W, w_dt)
    if metric == "wanda":
        a = np.asarray(aux, dtype=np.float32).reshape(1, -1)
        return rnd(np.abs(W) * rnd(np.sqrt(rnd(a + e, aux_dt)), aux_dt), promote(aux_dt, w_dt))
    if metric == "movement":
        pd = promote(w_dt, aux_dt)
        t = np.abs(rnd(W * np.asarray(aux, dtype=np.float32), pd))
        return rnd(t / np.float32(max(float(temperature), eps)), pd)
    return np.abs(W)


def score_stats(s: np.ndarray):
    """(mu, sigma) as the reference's f32 mean and std(unbiased=False) + 1e-6 (:1086-1087)."""
    d = s.astype(np.float64)
    mu = np.float32(d.mean())
    sigma = np.float32(np.float32(d.std()) + np.float32(1e-6))
    return mu, sigma


def znorm(s: np.ndarray, mu, sigma, sdt: str) -> np.ndarray:
    return rnd((s.astype(np.float32) - np.float32(mu)) / np.float32(sigma), sdt)


# ---------------------------------------------------------------------------
# schedules (sparse_modeling.py:932-985) and tau quantile (:987-1015)
# ---------------------------------------------------------------------------
def mask_update_period(step, period=10, switch_step=0, before=None, after=None) -> int:
    if switch_step > 0 and before is not None and after is not None:
        return int(before) if step < switch_step else int(after)
    return int(period)


def temperature(step, temp_init, temp_decay, temp_min, period, hard_type="match", block_temp_mult=2.0) -> float:
    K = max(1, int(period))
    updates = step // K
    init = float(temp_init)
    if hard_type in ("block_sparse16", "block_sparse32"):
        init *= float(block_temp_mult)
    return float(max(float(temp_min), init * (float(temp_decay) ** updates)))


def effective_sparsity(step, sparsity_ratio, warmup, hard_type="match") -> float:
    if warmup <= 0:
        return float(sparsity_ratio)
    r = min(1.0, max(0.0, step / max(1, warmup)))
    if hard_type in ("block_sparse16", "block_sparse32"):
        r = r * r * r
    return float(sparsity_ratio * r)


def beta_structural(step, start, end) -> float:
    if end <= start or step < start:
        return 0.0
    if step >= end:
        return 1.0
    t = float(step - start) / float(end - start)
    return float(3.0 * t * t - 2.0 * t * t * t)


def hardening_x(step, start, duration) -> float:
    """sparse_modeling.py:1603-1619."""
    if duration <= 0:
        return 0.0 if step >= start and start > 0 else 1.0
    if step < start:
        return 1.0
    if step >= start + duration:
        return 0.0
    progress = float(step - start) / float(max(1, duration))
    return max(0.0, min(1.0, 1.0 - progress))


def sorted_sample_indices(m: int, n: int, seed: int) -> np.ndarray:
    """The sorted tau sample the device draws (sf_sample_indices_sorted): m uniform draws from [0, n)
    in non-decreasing order, int64.  The reference draws torch.randint(0, n, (m,)) (:993); the
    quantile of a sample does not depend on its order.  E_j = -log((r_j + 1) 2^-53), r_j the top 53
    bits of splitmix64(seed, j), j = 0..m, held as round(E_j 2^32); S_k = E_0 + ... + E_k (exact
    integers); index k = floor(S_k / S_m * n), clamped below n.  (S_0 / S_m, ..., S_(m-1) / S_m) has
    the law of the order statistics of m independent U(0, 1) (Devroye 1986, ch. V.2).
    Pinned in tests/test_oracle_sampling.py by that law's closed-form moments, by the frequencies of
    numpy's own uniform integers and by exhaustive counts on tiny n."""
    from .hutchinson import splitmix64

    j = np.arange(m + 1, dtype=np.uint64)
    r = splitmix64(seed, j) >> np.uint64(11)
    u = (r.astype(np.float64) + 1.0) * 2.0 ** -53
    e = np.floor(-np.log(u) * 2.0 ** 32 + 0.5).astype(np.uint64)
    s = np.cumsum(e, dtype=np.uint64)
    idx = np.floor(s[:m].astype(np.float64) / float(s[m]) * float(n)).astype(np.int64)
    return np.minimum(idx, n - 1)


def quantile_linear(sample, q: float) -> np.float32:
    """torch.quantile(sample.float(), q) with linear interpolation (f32 ranks, torch lerp)."""
    v = np.sort(np.asarray(sample, dtype=np.float32).ravel())  # NaN sorts last
    n = v.size
    last = n - 1
    rank = np.float32(q) * np.float32(last)
    if np.isnan(v).any():
        rank = np.float32(last)
    lo = int(rank)
    hi = int(math.ceil(float(rank)))
    w = np.float32(rank - np.float32(lo))
    a, b = v[lo], v[hi]
    if abs(w) < 0.5:
        return np.float32(a + w * (b - a))
    return np.float32(b - (b - a) * (np.float32(1.0) - w))


# ---------------------------------------------------------------------------
# compute_gate_target (sparse_modeling.py:1018-1239) for mask_type
# unstructured / structured without block_sparse hard types
# ---------------------------------------------------------------------------
def gate_target(z: np.ndarray, sdt: str, mask_type: str, T: float, tau=None, N: int = 2, M: int = 4,
                structured_exact: bool = False, beta_s: float = 0.0, mask=None, frozen=None,
                hard_type: str = "match", sparsity: float = 0.0) -> np.ndarray:
    """G from the z-normalised scores z (already in the score dtype)."""
    denom = np.float32(np.float32(T) + np.float32(1e-8))
    rows, cols = z.shape
    block_core_ok = hard_type in BLOCK_SPARSE and all(block_core(z.shape, BLOCK_SIZE[hard_type]))
    if mask_type == "unstructured" and block_core_ok:  # :1122-1158: G per block from the blocks' RMS
        bs = BLOCK_SIZE[hard_type]
        of, inf = block_core(z.shape, bs)
        rms = block_rms(z, bs)
        tau_b = quantile_linear(rms.ravel(), sparsity)
        Gb = sigmoid_f32((rms - tau_b) / denom)
        G = np.ones_like(z, dtype=np.float32)
        G[:of, :inf] = rnd(block_expand(Gb, bs), sdt)
    elif mask_type == "unstructured":  # :1162
        G = rnd(sigmoid_f32((z - np.float32(tau)) / denom), sdt)
    elif mask_type == "structured":  # :1164-1185
        if cols % M != 0:
            raise AssertionError(f"in_features ({cols}) must be divisible by M ({M}).")
        g = z.reshape(rows, cols // M, M)
        if structured_exact:
            G = topk_keep(g, N).astype(np.float32).reshape(rows, cols)
        else:
            tg = kth_largest(g, N)[..., None]
            G = rnd(sigmoid_f32((g - tg) / denom), sdt).reshape(rows, cols)
    else:
        raise ValueError(f"Invalid mask_type: {mask_type}")
    if beta_s > 0.0 and hard_type not in BLOCK_SPARSE:  # :1199-1225
        full = (cols // M) * M
        if full > 0:
            target = G.copy()
            tk = topk_keep(z[:, :full].reshape(rows, full // M, M), N)
            target[:, :full] = tk.astype(np.float32).reshape(rows, full)
            G = rnd(np.float32(1.0 - beta_s) * G + np.float32(beta_s) * target, sdt)
    if frozen is not None:  # :1227-1229
        fz = np.asarray(frozen) != 0
        if fz.any():
            G = G.copy()
            G[fz] = rnd(np.asarray(mask, dtype=np.float32), sdt)[fz]
    return blockify(G, hard_type, sdt).astype(np.float32)  # :1237


# ---------------------------------------------------------------------------
# update_mask after the step gating (sparse_modeling.py:1288-1661)
# ---------------------------------------------------------------------------
def binarize_push(G: np.ndarray, d: float, sdt: str) -> np.ndarray:
    """Multiplicative push away from 0.5 (sparse_modeling.py:1576-1590; utils.py:437-446)."""
    if d == 0.0:
        return G
    lt, gt = G < 0.5, G > 0.5
    G = G.copy()
    G[lt] = rnd(G[lt] * np.float32(1.0 - d), sdt)
    G[gt] = rnd(G[gt] * np.float32(1.0 + d), sdt)
    return G


def ema(prev: np.ndarray, G: np.ndarray, sdt: str, mdt: str, mask_lr: float) -> np.ndarray:
    """mask.mul_(1 - a).add_(G, alpha=a).clamp_(0, 1) (sparse_modeling.py:1593; utils.py:448-449).

    add_ with alpha is a fused multiply-add; torch converts alpha to the op's
    dtype, so it is a bf16 alpha when mask and G are both bf16."""
    prev = np.asarray(prev, dtype=np.float32)
    alpha = np.float32(mask_lr) if F32 in (mdt, sdt) else round_bf16(np.float32(mask_lr))
    m1 = rnd(prev * np.float32(1.0 - mask_lr), mdt)
    m2 = rnd((np.asarray(G, np.float64) * np.float64(alpha) + m1.astype(np.float64)).astype(np.float32), mdt)
    return np.clip(m2, 0.0, 1.0).astype(np.float32)


def block_penalty_target(mode: str, G: np.ndarray, prev: np.ndarray, sparsity_ratio: float) -> np.ndarray:
    """Hard target of the block penalty modes, or None when the core is empty (-> 'mid').

    block16 (:1298-1347): top-k of G inside each 16x16 tile, k = round((1 - sr) 256).
    block_sparse16 / 32 (:1395-1529): the round((1 - sr) nblocks) blocks of largest mask mean."""
    bs = BLOCK_SIZE[mode]
    of, inf = block_core(G.shape, bs)
    if of == 0 or inf == 0:
        return None
    ob, ib = of // bs, inf // bs
    target = np.ones_like(G, dtype=np.float32)
    if mode == "block16":
        k = keep_count(1.0 - sparsity_ratio, bs * bs)
        keep = topk_keep_desc(block_tiles(G, bs), k).astype(np.float32)
        target[:of, :inf] = keep.reshape(ob, ib, bs, bs).transpose(0, 2, 1, 3).reshape(of, inf)
    else:
        k = keep_count(1.0 - sparsity_ratio, ob * ib)
        keep = topk_keep_desc(block_mean(prev, bs).ravel(), k).reshape(ob, ib)
        target[:of, :inf] = block_expand(keep, bs)
    return target


def update_mask(mask: np.ndarray, G: np.ndarray, sdt: str, mdt: str, mask_lr: float, penalty_mode: str = "none",
                penalty_coef: float = 0.0, N: int = 2, M: int = 4, binarize: float = 0.0, freeze_low: float = 0.0,
                freeze_high: float = 1.0, step: int = 0, frozen=None, hard_type: str = "nm_2_4",
                sparsity_ratio: float = 0.5):
    """Returns (new_mask, new_frozen_flags_or_None, flips).  G from gate_target."""
    prev = np.asarray(mask, dtype=np.float32).copy()
    G = np.asarray(G, dtype=np.float32).copy()
    rows, cols = prev.shape
    c = np.float32(penalty_coef)
    if penalty_coef != 0.0:
        mode = penalty_mode
        if mode in BLOCK_SIZE:
            target = block_penalty_target(mode, G, prev, sparsity_ratio)
            if target is None:
                mode = "mid"
            else:
                delta = rnd(rnd(prev, sdt) - target, sdt)
                G = rnd(G - rnd(c * delta, sdt), sdt)
        if mode == "nm_2_4" and (cols // 4) * 4 == 0:
            mode = "mid"
        if mode == "structured_topn" and cols % M != 0:
            mode = "mid"
        if mode in ("nm_2_4", "structured_topn"):  # :1350-1393, :1531-1565
            n = 2 if mode == "nm_2_4" else N
            full = (cols // 4) * 4
            target = np.ones_like(G)
            if full:
                target[:, :full] = topk_keep(G[:, :full].reshape(rows, full // 4, 4), n).reshape(rows, full)
            delta = rnd(rnd(prev, sdt) - target, sdt)
            G = rnd(G - rnd(c * delta, sdt), sdt)
        elif mode == "mid":  # :1567-1570
            pg = rnd(rnd(np.float32(1.0) - np.float32(2.0) * prev, mdt), sdt)
            G = rnd(G - rnd(c * pg, sdt), sdt)
        G = np.clip(G, 0.0, 1.0).astype(np.float32)
    G = binarize_push(G, binarize, sdt)
    new = ema(prev, G, sdt, mdt, mask_lr)
    new = blockify(new, hard_type, mdt)  # :1598-1601
    new_frozen = None
    if freeze_low > 0.0 or freeze_high < 1.0:  # :1621-1642
        f0 = new <= np.float32(freeze_low)
        f1 = new >= np.float32(freeze_high)
        new[f0] = 0.0
        applied = f0.copy()
        if step >= 2000:
            new[f1] = 1.0
            applied |= f1
        if frozen is not None:
            new_frozen = np.maximum(np.asarray(frozen, dtype=np.float32), applied.astype(np.float32))
    hp = hard_mask_from_soft(prev, hard_type, N, M, sparsity_ratio) > 0.5
    hn = hard_mask_from_soft(new, hard_type, N, M, sparsity_ratio) > 0.5
    return new, new_frozen, int((hp ^ hn).sum())


# ---------------------------------------------------------------------------
# layer-level compositions driven by a SparseLinearConfig-like dict
# ---------------------------------------------------------------------------
# Defaults of SparseLinearConfig (legacy/sparse_modeling.py:136-239).
CONFIG_DEFAULTS = dict(
    change_mask=True, mode="sparse_forward", mask_type="structured", mask_metric="hessian_obd",
    sparsity_ratio=0.5, N=2, M=4, beta=0.99, score_ema_beta=0.99, mask_update_period=10,
    mask_update_switch_step=0, mask_update_period_before=None, mask_update_period_after=None, mask_lr=0.10,
    mask_penalty_lr=None, mask_penalty_mode="mid", temp_init=1.0, temp_min=0.05, temp_decay=0.97,
    mask_binarize_decay=0.0, mask_hardening_start=1000, mask_hardening_duration=10000,
    sparsity_warmup_steps=100, tau_sample_size=262144, temperature=1.0, freeze_low=0.0, freeze_high=1.0,
    SLoRB=False, SLoRB_k=64, SLoRB_init_type="mean", trainable_projection=False, structured_exact=False,
    hard_mask_type="match", beta_structural_start=0, beta_structural_end=0, srste_decay=0.0,
    glu_joint_mask=False, weight_scaling=False,
)


def full_config(**kw) -> dict:
    c = dict(CONFIG_DEFAULTS)
    c.update(kw)
    return c


def _period(c, step):
    return mask_update_period(step, c["mask_update_period"], c["mask_update_switch_step"],
                              c["mask_update_period_before"], c["mask_update_period_after"])


def layer_schedule(c: dict, step: int) -> dict:
    """Host scalars of one step: T, sparsity, beta_s, hardening_x (sparse_modeling.py:932-985, :1603-1619)."""
    K = _period(c, step)
    return dict(
        K=K,
        T=temperature(step, c["temp_init"], c["temp_decay"], c["temp_min"], K, c["hard_mask_type"]),
        sparsity=effective_sparsity(step, c["sparsity_ratio"], c["sparsity_warmup_steps"], c["hard_mask_type"]),
        beta_s=beta_structural(step, c["beta_structural_start"], c["beta_structural_end"]),
        hx=hardening_x(step, c["mask_hardening_start"], c["mask_hardening_duration"]),
    )


def effective_hard_type(c: dict) -> str:
    h = c["hard_mask_type"] or "match"
    return c["mask_type"] if h == "match" else h


def effective_metric(c: dict, W, H) -> str:
    """The metric compute_gate_target evaluates: a Hessian metric whose hessian_diag is a placeholder falls
    back to W * W (hessian_obd) or |W| (hessian_ratio, hessian) (:1049-1068)."""
    metric = c["mask_metric"]
    if metric in ("hessian_obd", "hessian_ratio", "hessian") and (H is None or np.shape(H) != np.shape(W)):
        return "weight_squared" if metric == "hessian_obd" else "magnitude"
    return metric


def layer_gate_target(c: dict, step: int, W, H, mask, frozen, sample_idx, w_dt=F32, h_dt=F32, m_dt=F32, aux=None,
                      aux_dt=F32):
    """SparseLinear.compute_gate_target for mask_type unstructured / structured (non-block hard types).

    frozen: full flags tensor or None (placeholder).  sample_idx: indices of the tau
    sample (the reference draws them with torch.randint, :993).
    """
    if (not c["change_mask"]) or c["mask_type"] == "none":
        return np.ones_like(np.asarray(mask, dtype=np.float32))
    metric = effective_metric(c, W, H)
    s = scores(W, H, aux, metric, w_dt, h_dt, aux_dt, temperature=c["temperature"])
    sdt = score_dtype(metric, w_dt, h_dt, aux_dt)
    mu, sigma = score_stats(s)
    z = znorm(s, mu, sigma, sdt)
    sch = layer_schedule(c, step)
    tau = None
    if c["mask_type"] == "unstructured":
        flat = z.ravel()
        sample = flat[np.asarray(sample_idx)] if sample_idx is not None else flat
        tau = quantile_linear(sample, sch["sparsity"])
    return gate_target(z, sdt, c["mask_type"], sch["T"], tau, int(c["N"]), int(c["M"]), bool(c["structured_exact"]),
                       sch["beta_s"], mask, frozen, c["hard_mask_type"] or "match", sch["sparsity"])


def layer_update_mask(c: dict, step: int, W, H, mask, frozen, sample_idx, lambda_mid: float, w_dt=F32, h_dt=F32,
                      m_dt=F32, aux=None, aux_dt=F32):
    """SparseLinear.update_mask.  Returns (mask, frozen, flips, hardening_x) or None when the step is gated off."""
    if (not c["change_mask"]) or c["mask_type"] == "none":
        return None
    if step < int(c["sparsity_warmup_steps"]):
        return None
    K = max(1, _period(c, step))
    if step % K != 0:
        return None
    G = layer_gate_target(c, step, W, H, mask, frozen, sample_idx, w_dt, h_dt, m_dt, aux, aux_dt)
    sdt = score_dtype(effective_metric(c, W, H), w_dt, h_dt, aux_dt)
    pen_lr = float(c["mask_penalty_lr"]) if c["mask_penalty_lr"] is not None else float(c["mask_lr"])
    lam = float(lambda_mid or 0.0)
    mode = c["mask_penalty_mode"] or "mid"
    new, new_frozen, flips = update_mask(
        mask, G, sdt, m_dt, float(c["mask_lr"]), mode if lam != 0.0 else "none", pen_lr * lam, int(c["N"]),
        int(c["M"]), float(c["mask_binarize_decay"] or 0.0), float(c["freeze_low"]), float(c["freeze_high"]), step,
        frozen, effective_hard_type(c), float(c["sparsity_ratio"]))
    hx = layer_schedule(c, step)["hx"]
    return new, new_frozen, flips, hx


def joint_gate_target(c: dict, step: int, S, mask, frozen, sample_idx, m_dt=F32) -> np.ndarray:
    """_compute_joint_gate_target(module, scores, step) (utils.py:536-613) for a module of config c:
    z = ((S - mu) / sigma) in the mask dtype, the gate form (a mask_type other than structured behaves as
    unstructured; tau = quantile of z over the sample), the beta structural mix, the frozen override."""
    S = np.asarray(S, np.float32)
    if S.size == 0:
        return np.asarray(mask, np.float32)
    mu, sigma = score_stats(S)
    z = znorm(S, mu, sigma, m_dt)
    sch = layer_schedule(c, step)
    mtype = "structured" if c["mask_type"] == "structured" else "unstructured"
    N, M = int(c["N"]), int(c["M"])
    tau = None
    if mtype == "unstructured":
        flat = z.ravel()
        sample = flat[np.asarray(sample_idx)] if sample_idx is not None else flat
        tau = quantile_linear(sample, sch["sparsity"])
    return gate_target(z, m_dt, mtype, sch["T"], tau, N, M, bool(c["structured_exact"]), sch["beta_s"], mask, frozen)


def glu_joint_update(c: dict, step: int, Wg, Hg, Mg, Wu, Hu, Mu, frozen_g, sample_idx, lambda_mid: float,
                     w_dt=F32, h_dt=F32, m_dt=F32, aux_g=None, aux_u=None, aux_dt=F32):
    """_update_glu_joint_mask (utils.py:363-479) for one gate/up pair sharing config c (the gate's).

    Joint score S = score(gate) + score(up) in the score dtype (:415-420); z and G
    in the mask dtype (_compute_joint_gate_target, :536-613; a mask_type other than
    structured behaves as unstructured); the penalty compares G with the GATE mask
    (_apply_mid_penalty_to_gate, :615-643: structured_topn when cols % M == 0,
    else mid; any other mode only clamps); binarisation; the same G EMA'd into
    both masks; no freeze.  Returns (gate_mask, up_mask, flips_gate, flips_up,
    hardening_x) or None when the step is gated off.
    """
    if (not c["change_mask"]) or c["mask_type"] == "none":
        return None
    if step < int(c["sparsity_warmup_steps"]):
        return None
    K = max(1, _period(c, step))
    if step % K != 0:
        return None
    metric = c["mask_metric"]
    sdt = score_dtype(metric, w_dt, h_dt, aux_dt)
    sg = scores(Wg, Hg, aux_g, metric, w_dt, h_dt, aux_dt, temperature=c["temperature"])
    su = scores(Wu, Hu, aux_u, metric, w_dt, h_dt, aux_dt, temperature=c["temperature"])
    S = rnd(sg + su, sdt)
    sch = layer_schedule(c, step)
    N, M = int(c["N"]), int(c["M"])
    G = joint_gate_target(c, step, S, Mg, frozen_g, sample_idx, m_dt)
    Mg = np.asarray(Mg, np.float32)
    rows, cols = Mg.shape
    lam = float(lambda_mid or 0.0)
    if lam != 0.0:
        pen_lr = float(c["mask_penalty_lr"]) if c["mask_penalty_lr"] is not None else float(c["mask_lr"])
        coef = np.float32(pen_lr * lam)
        mode = c["mask_penalty_mode"] or "mid"
        if mode == "structured_topn" and cols % M != 0:
            mode = "mid"
        if mode == "structured_topn":
            target = topk_keep(G.reshape(rows, cols // M, M), N).astype(np.float32).reshape(rows, cols)
            G = rnd(G - rnd(coef * rnd(rnd(Mg, m_dt) - target, m_dt), m_dt), m_dt)
        elif mode == "mid":
            pg = rnd(rnd(np.float32(1.0) - np.float32(2.0) * Mg, m_dt), m_dt)
            G = rnd(G - rnd(coef * pg, m_dt), m_dt)
        G = np.clip(G, 0.0, 1.0).astype(np.float32)
    G = binarize_push(G, float(c["mask_binarize_decay"] or 0.0), m_dt)
    new_g = ema(Mg, G, m_dt, m_dt, float(c["mask_lr"]))
    new_u = ema(Mu, G, m_dt, m_dt, float(c["mask_lr"]))
    ht = effective_hard_type(c)
    fg = int(((hard_mask_from_soft(Mg, ht, N, M) > 0.5) ^ (hard_mask_from_soft(new_g, ht, N, M) > 0.5)).sum())
    fu = int(((hard_mask_from_soft(np.asarray(Mu, np.float32), ht, N, M) > 0.5)
              ^ (hard_mask_from_soft(new_u, ht, N, M) > 0.5)).sum())
    return new_g, new_u, fg, fu, sch["hx"]
