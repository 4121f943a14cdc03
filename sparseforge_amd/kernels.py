"""torch-tensor wrappers over the C ABI (include/sparseforge_amd.h).

Each function validates shapes/dtypes, takes raw device pointers from the
tensors, launches on torch's current stream of the tensors' device and
returns without synchronising.  Workspaces come from torch's caching
allocator; the library itself never allocates.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib as L
from . import profiling as _prof


def _written(*ts) -> None:
    """Bump the version counter of tensors a kernel wrote in place, as a torch in-place op would: caches
    keyed on a mask's version (the forward's effective mask) then see the write."""
    for t in ts:
        if t is not None:
            torch.autograd.graph.increment_version(t)


def _ws(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------
# hard projections (SparseLinear._hard_mask_from_soft, sparse_modeling.py:510-735)
# ---------------------------------------------------------------------------
def hard_mask(soft: torch.Tensor, kind: int, n_keep: int = 2, m_group: int = 4,
              out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    dev = L.require_device(soft)
    if soft.dim() != 2:
        raise ValueError("hard_mask expects a 2-D soft mask")
    if out is None:
        out = torch.empty_like(soft, dtype=out_dtype or soft.dtype)
    L.require_device(out)
    rows, cols = soft.shape
    with _prof.region("sf_hard_mask", soft.numel() * (soft.element_size() + out.element_size()), "B", dev):
        L.check(
            L.lib().sf_hard_mask(L.ptr(soft), L.dtype_code(soft), L.ptr(out), L.dtype_code(out), rows, cols,
                                 kind, n_keep, m_group, L.stream(dev)),
            "sf_hard_mask",
        )
    return out


def hard_flip_count(prev: torch.Tensor, now: torch.Tensor, kind: int, n_keep: int = 2, m_group: int = 4,
                    counter: torch.Tensor | None = None) -> torch.Tensor:
    """Device int64[1] count of positions where hard(prev) != hard(now)."""
    dev = L.require_device(prev, now)
    if prev.shape != now.shape or prev.dtype != now.dtype or prev.dim() != 2:
        raise ValueError("hard_flip_count: prev/now must be 2-D with equal shape and dtype")
    if counter is None:
        counter = torch.zeros(1, dtype=torch.int64, device=dev)
    rows, cols = prev.shape
    L.check(
        L.lib().sf_hard_flip_count(L.ptr(prev), L.ptr(now), L.dtype_code(prev), rows, cols, kind, n_keep,
                                   m_group, L.ptr(counter), L.stream(dev)),
        "sf_hard_flip_count",
    )
    return counter


# ---------------------------------------------------------------------------
# gate target and fused mask update (sparse_modeling.py:1018-1666)
# ---------------------------------------------------------------------------
@dataclass
class MaskOperands:
    """Device tensors of one layer's mask state."""

    weight: torch.Tensor
    mask: torch.Tensor
    hessian: torch.Tensor | None = None   # hessian_diag [out, in] (None if placeholder)
    aux: torch.Tensor | None = None       # scaler_row [in] (wanda) or grad_ema [out, in] (movement)
    frozen: torch.Tensor | None = None    # frozen_mask_flags [out, in] (None if placeholder)

    def device(self) -> torch.device:
        dev = L.require_device(self.weight, self.mask, self.hessian, self.aux, self.frozen)
        shape = tuple(self.weight.shape)
        if self.weight.dim() != 2:
            raise ValueError("mask ops expect a 2-D weight")
        for name, t in (("mask", self.mask), ("hessian_diag", self.hessian), ("frozen_mask_flags", self.frozen)):
            if t is not None and tuple(t.shape) != shape:
                raise ValueError(f"{name} shape {tuple(t.shape)} != weight shape {shape}")
        if self.aux is not None and tuple(self.aux.shape) not in (shape, (shape[1],)):
            raise ValueError(f"aux shape {tuple(self.aux.shape)} fits neither {shape} nor ({shape[1]},)")
        return dev

    def dt(self, t: torch.Tensor | None) -> int:
        return L.dtype_code(t) if t is not None else L.DT_F32

    def score_bytes(self) -> int:
        """Bytes of the score operands (W, H, aux), each read once."""
        return sum(t.numel() * t.element_size() for t in (self.weight, self.hessian, self.aux) if t is not None)


def score_stats(p: L.MaskParams, ops: MaskOperands, workspace: torch.Tensor | None = None) -> torch.Tensor:
    dev = ops.device()
    ws = workspace if workspace is not None else _ws(L.lib().sf_mask_workspace_size(p.rows, p.cols, 0), dev)
    stats = torch.empty(2, dtype=torch.float32, device=dev)
    with _prof.region("sf_score_stats", ops.score_bytes(), "B", dev):
        L.check(
            L.lib().sf_score_stats(ctypes.byref(p), L.ptr(ops.weight), ops.dt(ops.weight), L.ptr(ops.hessian),
                                   ops.dt(ops.hessian), L.ptr(ops.aux), ops.dt(ops.aux), L.ptr(stats), L.ptr(ws),
                                   ws.numel(), L.stream(dev)),
            "sf_score_stats",
        )
    return stats


def sample_indices(sample_size: int, n: int, seed: int, device: torch.device) -> torch.Tensor:
    idx = torch.empty(sample_size, dtype=torch.int64, device=device)
    L.check(L.lib().sf_sample_indices(L.ptr(idx), sample_size, n, seed & ((1 << 64) - 1), L.stream(device)),
            "sf_sample_indices")
    return idx


def sample_indices_sorted(sample_size: int, ns, seeds, device: torch.device) -> torch.Tensor:
    """[len(ns), sample_size] int64: row c holds sample_size uniform draws from [0, ns[c]) in
    non-decreasing order (sf_sample_indices_sorted), from the counter generator seeded by seeds[c]."""
    ns, seeds = [int(v) for v in ns], [int(v) & ((1 << 64) - 1) for v in seeds]
    if len(ns) != len(seeds):
        raise ValueError("one seed per list")
    count = len(ns)
    idx = torch.empty((count, sample_size), dtype=torch.int64, device=device)
    if count == 0 or sample_size == 0:
        return idx
    ws = _ws(L.lib().sf_sample_indices_sorted_workspace_size(sample_size, count), device)
    n_arr = (ctypes.c_int64 * count)(*ns)
    s_arr = (ctypes.c_uint64 * count)(*seeds)
    L.check(L.lib().sf_sample_indices_sorted(L.ptr(idx), sample_size, n_arr, s_arr, count, L.ptr(ws), ws.numel(),
                                             L.stream(device)),
            "sf_sample_indices_sorted")
    return idx


def tau_quantile(p: L.MaskParams, ops: MaskOperands, stats: torch.Tensor, q: float,
                 sample_idx: torch.Tensor | None) -> torch.Tensor:
    dev = ops.device()
    if sample_idx is not None:
        L.require_device(sample_idx)
        if sample_idx.dim() != 1:
            raise ValueError("sample indices must be 1-D")
        if sample_idx.dtype != torch.int64:
            raise TypeError("sample indices must be int64")
        m = sample_idx.numel()
    else:
        m = p.rows * p.cols
    ws = _ws(L.lib().sf_mask_workspace_size(p.rows, p.cols, m), dev)
    tau = torch.empty(1, dtype=torch.float32, device=dev)
    with _prof.region("sf_tau_quantile", m * 8, "B", dev):
        L.check(
            L.lib().sf_tau_quantile(ctypes.byref(p), L.ptr(ops.weight), ops.dt(ops.weight), L.ptr(ops.hessian),
                                    ops.dt(ops.hessian), L.ptr(ops.aux), ops.dt(ops.aux), L.ptr(stats),
                                    L.ptr(sample_idx), m, float(q), L.ptr(tau), L.ptr(ws), ws.numel(),
                                    L.stream(dev)),
            "sf_tau_quantile",
        )
    return tau


def tau_quantile_noalloc(p: L.MaskParams, ops: MaskOperands, stats: torch.Tensor, q: float,
                         sample_idx: torch.Tensor | None, out: torch.Tensor | None = None) -> torch.Tensor:
    """tau_quantile through sf_tau_quantile_noalloc: the library's static scratch, no workspace.

    `out` (device float[1]) lets a caller that cannot allocate pass the output
    too.  Calls that overlap on one GPU race on the shared scratch."""
    dev = ops.device()
    if sample_idx is not None:
        L.require_device(sample_idx)
        if sample_idx.dim() != 1 or sample_idx.dtype != torch.int64:
            raise TypeError("sample indices must be a 1-D int64 tensor")
        m = sample_idx.numel()
    else:
        m = p.rows * p.cols
    if m > L.TAU_NOALLOC_MAX_SAMPLE:
        raise ValueError(f"tau sample of {m} elements exceeds the static scratch maximum {L.TAU_NOALLOC_MAX_SAMPLE}")
    tau = out if out is not None else torch.empty(1, dtype=torch.float32, device=dev)
    L.check(
        L.lib().sf_tau_quantile_noalloc(ctypes.byref(p), L.ptr(ops.weight), ops.dt(ops.weight), L.ptr(ops.hessian),
                                        ops.dt(ops.hessian), L.ptr(ops.aux), ops.dt(ops.aux), L.ptr(stats),
                                        L.ptr(sample_idx), m, float(q), L.ptr(tau), L.stream(dev)),
        "sf_tau_quantile_noalloc",
    )
    return tau


def gate_target(p: L.MaskParams, ops: MaskOperands, stats: torch.Tensor, tau: torch.Tensor | None,
                g_dtype: torch.dtype) -> torch.Tensor:
    dev = ops.device()
    G = torch.empty(p.rows, p.cols, dtype=g_dtype, device=dev)
    L.check(
        L.lib().sf_gate_target(ctypes.byref(p), L.ptr(ops.weight), ops.dt(ops.weight), L.ptr(ops.hessian),
                               ops.dt(ops.hessian), L.ptr(ops.aux), ops.dt(ops.aux), L.ptr(ops.mask),
                               ops.dt(ops.mask), L.ptr(ops.frozen), ops.dt(ops.frozen), L.ptr(stats), L.ptr(tau),
                               L.ptr(G), L.dtype_code(G), L.stream(dev)),
        "sf_gate_target",
    )
    return G


def update_mask(p: L.MaskParams, ops: MaskOperands, stats: torch.Tensor, tau: torch.Tensor | None,
                flips: torch.Tensor | None) -> None:
    dev = ops.device()
    # W, H, aux read once; mask read and written; frozen flags read and written when freezing
    nbytes = ops.score_bytes() + 2 * ops.mask.numel() * ops.mask.element_size()
    if ops.frozen is not None and p.apply_freeze:
        nbytes += 2 * ops.frozen.numel() * ops.frozen.element_size()
    with _prof.region("sf_update_mask", nbytes, "B", dev):
        L.check(
            L.lib().sf_update_mask(ctypes.byref(p), L.ptr(ops.weight), ops.dt(ops.weight), L.ptr(ops.hessian),
                                   ops.dt(ops.hessian), L.ptr(ops.aux), ops.dt(ops.aux), L.ptr(ops.mask),
                                   ops.dt(ops.mask), L.ptr(ops.frozen), ops.dt(ops.frozen), L.ptr(stats),
                                   L.ptr(tau), L.ptr(flips), L.stream(dev)),
            "sf_update_mask",
        )
    _written(ops.mask, ops.frozen)


@dataclass
class MaskJob:
    """One layer of a batched mask update: operands, tau sample and the device outputs."""

    ops: MaskOperands
    sample_idx: torch.Tensor | None  # tau sample indices (None: every element)
    stats: torch.Tensor              # f32 [2], written
    tau: torch.Tensor | None         # f32 [1], written (unstructured gate)
    flips: torch.Tensor | None       # int64 [1], incremented


def multi_workspace(jobs: list[MaskJob], device: torch.device) -> torch.Tensor:
    table = _layer_table(jobs)
    return _ws(L.lib().sf_update_mask_multi_workspace_size(table, len(jobs)), device)


def _layer_table(jobs: list[MaskJob]):
    table = (L.MaskLayer * max(len(jobs), 1))()
    for i, j in enumerate(jobs):
        o = j.ops
        rows, cols = o.weight.shape
        e = table[i]
        e.rows, e.cols = rows, cols
        e.W, e.H, e.aux = L.ptr(o.weight), L.ptr(o.hessian), L.ptr(o.aux)
        e.mask, e.frozen = L.ptr(o.mask), L.ptr(o.frozen)
        e.sample_idx = L.ptr(j.sample_idx)
        e.sample_size = j.sample_idx.numel() if j.sample_idx is not None else rows * cols
        e.stats, e.tau, e.flips = L.ptr(j.stats), L.ptr(j.tau), L.ptr(j.flips)
    return table


def update_mask_multi(p: L.MaskParams, q: float, jobs: list[MaskJob], stages: int = L.MULTI_ALL,
                      workspace: torch.Tensor | None = None) -> None:
    """sf_score_stats + sf_tau_quantile(q) + sf_update_mask of many layers whose parameters differ only in
    shape (p.rows / p.cols are ignored), in a few launches per 28 layers; outputs equal the single-layer
    calls' bit for bit.  Every layer's tensors share one dtype per operand."""
    if not jobs:
        return
    dev = jobs[0].ops.device()
    first = jobs[0].ops
    dts = [first.dt(t) for t in (first.weight, first.hessian, first.aux, first.mask, first.frozen)]
    nbytes = 0
    for j in jobs:
        o = j.ops
        if o.device() != dev:
            raise ValueError("update_mask_multi: every layer must live on one device")
        for t, want, name in ((o.weight, dts[0], "weight"), (o.hessian, dts[1], "hessian_diag"),
                              (o.aux, dts[2], "aux"), (o.mask, dts[3], "mask"), (o.frozen, dts[4], "frozen")):
            if t is not None and o.dt(t) != want:
                raise ValueError(f"update_mask_multi: {name} dtypes differ between layers")
        L.require_device(o.weight, j.stats, j.tau, j.flips, j.sample_idx)
        if j.sample_idx is not None and (j.sample_idx.dim() != 1 or j.sample_idx.dtype != torch.int64):
            raise TypeError("sample indices must be a 1-D int64 tensor")
        # algorithmic bytes: the statistics read the score operands, the update reads them again and
        # reads + writes the mask (and the frozen flags when freezing)
        if stages & L.MULTI_STATS:
            nbytes += o.score_bytes()
        if stages & L.MULTI_UPDATE:
            nbytes += o.score_bytes() + 2 * o.mask.numel() * o.mask.element_size()
            if o.frozen is not None and p.apply_freeze:
                nbytes += 2 * o.frozen.numel() * o.frozen.element_size()
    table = _layer_table(jobs)
    ws = workspace if workspace is not None else _ws(L.lib().sf_update_mask_multi_workspace_size(table, len(jobs)), dev)
    with _prof.region("sf_update_mask_multi", nbytes, "B", dev):
        L.check(
            L.lib().sf_update_mask_multi(ctypes.byref(p), float(q), table, len(jobs), int(stages), *dts, L.ptr(ws),
                                         ws.numel(), L.stream(dev)),
            "sf_update_mask_multi",
        )
    if stages & L.MULTI_UPDATE:
        for j in jobs:
            _written(j.ops.mask, j.ops.frozen)


# ---------------------------------------------------------------------------
# block hard types and block_sparse masks (sparse_modeling.py:460-507, :537-718,
# :1100-1158, :1237, :1298-1529, :1598-1601)
# ---------------------------------------------------------------------------
def block_stat(x: torch.Tensor, bs: int, stat: int) -> torch.Tensor:
    """Per-block mean (L.BLOCK_MEAN) or RMS (L.BLOCK_RMS) of the core of x: f32 [(rows//bs) * (cols//bs)]."""
    dev = L.require_device(x)
    if x.dim() != 2:
        raise ValueError("block_stat expects a 2-D tensor")
    x = x.contiguous()
    rows, cols = x.shape
    out = torch.empty((rows // bs) * (cols // bs), dtype=torch.float32, device=dev)
    with _prof.region("sf_block_stat", x.numel() * x.element_size(), "B", dev):
        L.check(L.lib().sf_block_stat(L.ptr(x), L.dtype_code(x), rows, cols, bs, stat, L.ptr(out), L.stream(dev)),
                "sf_block_stat")
    return out


def topk_keep(v: torch.Tensor, k: int) -> torch.Tensor:
    """f32 flags of the entries torch.topk(v, k) keeps for a 1-D f32 tensor (equal values as torch's
    CPU selection keeps them)."""
    dev = L.require_device(v)
    if v.dim() != 1 or v.dtype != torch.float32:
        raise ValueError("topk_keep expects a 1-D float32 tensor")
    keep = torch.empty_like(v)
    wb = L.lib().sf_topk_keep_workspace_size(v.numel())
    ws = torch.empty(max(wb, 16), dtype=torch.uint8, device=dev)
    L.check(L.lib().sf_topk_keep(L.ptr(v), v.numel(), int(k), L.ptr(keep), L.ptr(ws), wb, L.stream(dev)),
            "sf_topk_keep")
    return keep


def tile_topk(x: torch.Tensor, k: int, out_dtype: torch.dtype) -> torch.Tensor:
    """block16 projection: top-k of each 16 x 16 tile of the core -> 1, rest 0, outside the core 1."""
    dev = L.require_device(x)
    x = x.contiguous()
    rows, cols = x.shape
    out = torch.empty(rows, cols, dtype=out_dtype, device=dev)
    with _prof.region("sf_tile_topk", x.numel() * (x.element_size() + out.element_size()), "B", dev):
        L.check(L.lib().sf_tile_topk(L.ptr(x), L.dtype_code(x), rows, cols, 16, int(k), L.ptr(out),
                                     L.dtype_code(out), L.stream(dev)), "sf_tile_topk")
    return out


def block_fill(bvals: torch.Tensor | None, out: torch.Tensor, bs: int, tau: torch.Tensor | None = None,
               temperature: float = 0.0, edge_val: float | None = None, ov_src: torch.Tensor | None = None,
               ov_flags: torch.Tensor | None = None) -> torch.Tensor:
    """out[core] = bvals[block] (or sigmoid((b - tau) / (T + 1e-8)) with tau), cast to out's dtype, in place.

    edge_val None leaves the elements outside the core unchanged; ov_flags != 0 selects ov_src instead."""
    dev = L.require_device(out, bvals, tau, ov_src, ov_flags)
    if not out.is_contiguous() or out.dim() != 2:
        raise ValueError("block_fill writes a contiguous 2-D tensor")
    rows, cols = out.shape
    for t in (ov_src, ov_flags):
        if t is not None and (tuple(t.shape) != (rows, cols) or not t.is_contiguous()):
            raise ValueError("override operands must be contiguous and shaped like out")
    L.check(L.lib().sf_block_fill(L.ptr(bvals), rows, cols, bs, L.ptr(tau), float(temperature), L.ptr(out),
                                  L.dtype_code(out), int(edge_val is not None),
                                  float(edge_val if edge_val is not None else 0.0), L.ptr(ov_src),
                                  L.dtype_code(ov_src) if ov_src is not None else L.DT_F32, L.ptr(ov_flags),
                                  L.dtype_code(ov_flags) if ov_flags is not None else L.DT_F32, L.stream(dev)),
            "sf_block_fill")
    _written(out)
    return out


def apply_gate(p: L.MaskParams, G: torch.Tensor, target: torch.Tensor | None, mask: torch.Tensor,
               frozen: torch.Tensor | None, do_freeze: bool) -> None:
    dev = L.require_device(G, target, mask, frozen)
    nbytes = G.numel() * G.element_size() + 2 * mask.numel() * mask.element_size()
    if target is not None:
        nbytes += target.numel() * target.element_size()
    with _prof.region("sf_apply_gate", nbytes, "B", dev):
        L.check(L.lib().sf_apply_gate(ctypes.byref(p), L.ptr(G), L.ptr(target),
                                      L.dtype_code(target) if target is not None else L.DT_F32, L.ptr(mask),
                                      L.dtype_code(mask), L.ptr(frozen),
                                      L.dtype_code(frozen) if frozen is not None else L.DT_F32, int(do_freeze),
                                      L.stream(dev)), "sf_apply_gate")
    _written(mask, frozen)


def freeze_mask(p: L.MaskParams, mask: torch.Tensor, frozen: torch.Tensor | None) -> None:
    dev = L.require_device(mask, frozen)
    L.check(L.lib().sf_freeze_mask(ctypes.byref(p), L.ptr(mask), L.dtype_code(mask), L.ptr(frozen),
                                   L.dtype_code(frozen) if frozen is not None else L.DT_F32, L.stream(dev)),
            "sf_freeze_mask")
    _written(mask, frozen)


# ---------------------------------------------------------------------------
# GLU gate/up joint update (legacy/utils.py:363-643)
# ---------------------------------------------------------------------------
def importance_scores(p: L.MaskParams, ops: MaskOperands, s_dtype: torch.dtype) -> torch.Tensor:
    """One layer's importance scores in s_dtype (sf_importance_scores)."""
    dev = ops.device()
    S = torch.empty(ops.weight.shape, dtype=s_dtype, device=dev)
    with _prof.region("sf_importance_scores", ops.score_bytes() + S.numel() * S.element_size(), "B", dev):
        L.check(L.lib().sf_importance_scores(ctypes.byref(p), L.ptr(ops.weight), ops.dt(ops.weight),
                                             L.ptr(ops.hessian), ops.dt(ops.hessian), L.ptr(ops.aux), ops.dt(ops.aux),
                                             L.ptr(S), L.dtype_code(S), L.stream(dev)),
                "sf_importance_scores")
    return S


def joint_scores(pg: L.MaskParams, gate: MaskOperands, pu: L.MaskParams, up: MaskOperands,
                 s_dtype: torch.dtype) -> torch.Tensor:
    """S = score(gate) + score(up), rounded in s_dtype."""
    dev = L.require_device(gate.weight, up.weight)
    gate.device()
    up.device()
    if gate.weight.shape != up.weight.shape:
        raise ValueError(f"gate {tuple(gate.weight.shape)} and up {tuple(up.weight.shape)} shapes differ")
    for a, b, what in ((gate.weight, up.weight, "weight"), (gate.hessian, up.hessian, "hessian_diag"),
                       (gate.aux, up.aux, "aux")):
        if a is not None and b is not None and a.dtype != b.dtype:
            raise NotImplementedError(f"joint scores with gate/up {what} dtypes {a.dtype} / {b.dtype}")
    hd = gate.hessian if gate.hessian is not None else up.hessian
    ad = gate.aux if gate.aux is not None else up.aux
    S = torch.empty_like(gate.weight, dtype=s_dtype)
    with _prof.region("sf_joint_scores", gate.score_bytes() + up.score_bytes() + S.numel() * S.element_size(), "B",
                      dev):
        L.check(L.lib().sf_joint_scores(ctypes.byref(pg), L.ptr(gate.weight), L.ptr(gate.hessian), L.ptr(gate.aux),
                                        ctypes.byref(pu), L.ptr(up.weight), L.ptr(up.hessian), L.ptr(up.aux),
                                        L.dtype_code(gate.weight), gate.dt(hd), gate.dt(ad), L.ptr(S),
                                        L.dtype_code(S), L.stream(dev)),
                "sf_joint_scores")
    return S


def glu_update_masks(p: L.MaskParams, S: torch.Tensor, gate_mask: torch.Tensor, up_mask: torch.Tensor,
                     gate_frozen: torch.Tensor | None, stats: torch.Tensor, tau: torch.Tensor | None,
                     up_hard_kind: int, up_hard_n: int, gate_flips: torch.Tensor | None,
                     up_flips: torch.Tensor | None) -> None:
    dev = L.require_device(S, gate_mask, up_mask, gate_frozen, stats, tau, gate_flips, up_flips)
    for name, t in (("up mask", up_mask), ("gate mask", gate_mask), ("frozen_mask_flags", gate_frozen)):
        if t is not None and t.shape != S.shape:
            raise ValueError(f"{name} shape {tuple(t.shape)} != score shape {tuple(S.shape)}")
    if gate_mask.dtype != up_mask.dtype:
        raise NotImplementedError(f"joint update with gate/up mask dtypes {gate_mask.dtype} / {up_mask.dtype}")
    nbytes = S.numel() * (S.element_size() + 4 * gate_mask.element_size())
    with _prof.region("sf_glu_update_masks", nbytes, "B", dev):
        L.check(L.lib().sf_glu_update_masks(ctypes.byref(p), L.ptr(S), L.dtype_code(S), L.ptr(gate_mask),
                                            L.ptr(up_mask), L.dtype_code(gate_mask), L.ptr(gate_frozen),
                                            L.dtype_code(gate_frozen) if gate_frozen is not None else L.DT_F32,
                                            L.ptr(stats), L.ptr(tau), up_hard_kind, up_hard_n, L.ptr(gate_flips),
                                            L.ptr(up_flips), L.stream(dev)),
                "sf_glu_update_masks")
    _written(gate_mask, up_mask, gate_frozen)


# ---------------------------------------------------------------------------
# mask statistics and penalties (legacy/utils.py :876-1234, :2069-2280)
# ---------------------------------------------------------------------------
def mask_stats_workspace(device: torch.device) -> torch.Tensor:
    return _ws(L.lib().sf_mask_stats_workspace_size(), device)


def mask_stats(mask: torch.Tensor, out: torch.Tensor, tail_col: int = 0, eps: float = 1e-8,
               workspace: torch.Tensor | None = None) -> torch.Tensor:
    """out (f64 [MSTAT_COUNT], device) = the fused sums of one mask (rows x cols; a 1-D mask is one row)."""
    dev = L.require_device(mask, out)
    if out.dtype != torch.float64 or out.numel() != L.MSTAT_COUNT:
        raise ValueError("mask_stats: out must be a contiguous float64 tensor of MSTAT_COUNT elements")
    if mask.dim() not in (1, 2):
        raise ValueError("mask_stats expects a 1-D or 2-D mask")
    rows, cols = (1, mask.numel()) if mask.dim() == 1 else mask.shape
    ws = workspace if workspace is not None else mask_stats_workspace(dev)
    with _prof.region("sf_mask_stats", mask.numel() * mask.element_size(), "B", dev):
        L.check(L.lib().sf_mask_stats(L.ptr(mask), L.dtype_code(mask), rows, cols, int(tail_col), float(eps),
                                      L.ptr(out), L.ptr(ws), ws.numel(), L.stream(dev)), "sf_mask_stats")
    return out


def mask_hist(mask: torch.Tensor, idx: torch.Tensor, bins: int, lo: float, hi: float,
              hist: torch.Tensor) -> torch.Tensor:
    """hist (int64 [bins], device) += torch.histc-style counts of mask.flatten()[idx] over [lo, hi]."""
    dev = L.require_device(mask, idx, hist)
    if idx.dtype != torch.int64 or hist.dtype != torch.int64 or hist.numel() != int(bins):
        raise ValueError("mask_hist: idx and hist must be int64, hist of `bins` elements")
    L.check(L.lib().sf_mask_hist(L.ptr(mask), L.dtype_code(mask), mask.numel(), L.ptr(idx), idx.numel(), int(bins),
                                 float(lo), float(hi), L.ptr(hist), L.stream(dev)), "sf_mask_hist")
    return hist


def keep_split_sum(v: torch.Tensor, keep: torch.Tensor) -> torch.Tensor:
    """f64 [2] (device): sum of v where keep != 0, sum of the rest."""
    dev = L.require_device(v, keep)
    if v.dtype != torch.float32 or keep.dtype != torch.float32 or v.shape != keep.shape or v.dim() != 1:
        raise ValueError("keep_split_sum expects two 1-D float32 tensors of one shape")
    out = torch.empty(2, dtype=torch.float64, device=dev)
    L.check(L.lib().sf_keep_split_sum(L.ptr(v), L.ptr(keep), v.numel(), L.ptr(out), L.stream(dev)),
            "sf_keep_split_sum")
    return out


# ---------------------------------------------------------------------------
# Cross-layer overlap of the mask updates
# ---------------------------------------------------------------------------
_SIDE_STREAMS: dict = {}


class LayerPipeline:
    """Spread independent per-layer mask updates over a few side streams.

    A layer's update is a chain of kernels (score statistics, the tau
    selection passes, the fused update) whose middle part is latency-bound;
    on separate streams the chains of different layers overlap, so those
    kernels hide behind the memory-bound ones of other layers.  The side
    streams first wait for the current stream's work, and join() makes the
    current stream wait for them.  Streams keep the default priority.
    """

    def __init__(self, device: torch.device, n: int = 4):
        key = (device.index, n)
        if key not in _SIDE_STREAMS:
            _SIDE_STREAMS[key] = [torch.cuda.Stream(device=device) for _ in range(n)]
        self.main = torch.cuda.current_stream(device)
        self.streams = _SIDE_STREAMS[key]
        start = torch.cuda.Event()
        start.record(self.main)
        for st in self.streams:
            st.wait_event(start)
        self.i = 0

    def next(self):
        """Context manager: run the next layer's update on the next side stream."""
        st = self.streams[self.i % len(self.streams)]
        self.i += 1
        return torch.cuda.stream(st)

    def join(self) -> None:
        for st in self.streams:
            ev = torch.cuda.Event()
            ev.record(st)
            self.main.wait_event(ev)
