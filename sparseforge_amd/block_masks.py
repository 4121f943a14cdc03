"""Block hard types and block_sparse soft masks on the HIP kernels.

Reference: legacy/sparse_modeling.py -- _blockify_tensor (:460-507), the
block16 / block_sparse16 / block_sparse32 projections of _hard_mask_from_soft
(:537-718), the block-level gate of compute_gate_target (:1100-1158) and its
final blockify (:1237), the block penalty modes of update_mask (:1298-1529)
and the mask blockify after the EMA (:1598-1601).

Blocks are the bs x bs tiles of the fully covered core
[:rows // bs * bs, :cols // bs * bs]; elements outside it are left alone by
blockify and are 1 in hard masks, penalty targets and the block gate.  Equal
values are kept exactly as torch.topk's CPU kernel keeps them (its libstdc++
nth_element / partial_sort selection, reproduced step for step by
sf_topk_keep and sf_tile_topk), e.g. for the initial all-ones mask.
"""
from __future__ import annotations

import torch

from . import _lib as L
from . import kernels as K

BLOCK_SIZE = {"block16": 16, "block_sparse16": 16, "block_sparse32": 32}
BLOCK_SPARSE = ("block_sparse16", "block_sparse32")


def keep_count(frac_kept: float, total: int) -> int:
    """int(round((1 - sr) * total)) clipped to [0, total], as the reference computes keep_k / keep_blocks."""
    return max(0, min(total, int(round(frac_kept * total))))


def core_blocks(shape, bs: int):
    rows, cols = shape
    return rows // bs, cols // bs


def hard_mask(soft: torch.Tensor, hard_type: str, sparsity_ratio: float,
              out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """_hard_mask_from_soft for block16 (:537-575) and block_sparse16 / 32 (:607-718)."""
    bs = BLOCK_SIZE[hard_type]
    soft = soft.contiguous()
    dt = out_dtype or soft.dtype
    ob, ib = core_blocks(soft.shape, bs)
    if hard_type == "block16":
        return K.tile_topk(soft, keep_count(1.0 - sparsity_ratio, bs * bs), dt)
    out = torch.empty(soft.shape, dtype=dt, device=soft.device)
    if ob == 0 or ib == 0:
        return K.block_fill(None, out, bs, edge_val=1.0)
    rms = K.block_stat(soft, bs, L.BLOCK_RMS)
    keep = K.topk_keep(rms, keep_count(1.0 - sparsity_ratio, ob * ib))
    return K.block_fill(keep, out, bs, edge_val=1.0)


def blockify_(t: torch.Tensor, hard_type: str) -> torch.Tensor:
    """_blockify_tensor in place: every core block takes its mean (f32), cast to t's dtype."""
    if hard_type not in BLOCK_SPARSE or t.dim() != 2:
        return t
    bs = BLOCK_SIZE[hard_type]
    ob, ib = core_blocks(t.shape, bs)
    if ob == 0 or ib == 0:
        return t
    means = K.block_stat(t, bs, L.BLOCK_MEAN)
    return K.block_fill(means, t, bs)


def block_gate(z: torch.Tensor, hard_type: str, sparsity: float, temperature: float, mask: torch.Tensor,
               frozen: torch.Tensor | None) -> torch.Tensor:
    """The block_sparse branch of the unstructured gate (:1122-1154) plus the frozen override (:1227-1229).

    z: z-normalised scores in the score dtype.  The block RMS of z is thresholded at its own
    torch.quantile(q = sparsity) over all blocks; G = sigmoid((rms - tau_b) / (T + 1e-8)) per block,
    1 outside the core, mask where frozen."""
    bs = BLOCK_SIZE[hard_type]
    ob, ib = core_blocks(z.shape, bs)
    rms = K.block_stat(z, bs, L.BLOCK_RMS)
    v = rms.view(1, -1)
    p = L.MaskParams()
    p.rows, p.cols = 1, ob * ib
    p.metric = L.METRIC["hessian"]  # the "score" of an entry is the entry itself
    p.score_dtype = L.DT_F32
    ops = K.MaskOperands(weight=v, mask=v, hessian=v)
    unit = torch.tensor([0.0, 1.0], dtype=torch.float32, device=z.device)  # z = (v - 0) / 1 = v
    tau_b = K.tau_quantile(p, ops, unit, float(sparsity), None)
    G = torch.empty_like(z)
    return K.block_fill(rms, G, bs, tau=tau_b, temperature=temperature, edge_val=1.0,
                        ov_src=mask if frozen is not None else None, ov_flags=frozen)


def penalty_target(mode: str, G: torch.Tensor, mask: torch.Tensor, sparsity_ratio: float) -> torch.Tensor | None:
    """Hard target of the block penalty modes in G's dtype, or None when the core is empty
    (the reference then falls back to 'mid').

    block16 (:1298-1347): top-k of G in each 16 x 16 tile, k = round((1 - sr) 256).
    block_sparse16 / 32 (:1395-1529): the round((1 - sr) nblocks) blocks of largest mask mean."""
    bs = BLOCK_SIZE[mode]
    ob, ib = core_blocks(G.shape, bs)
    if ob == 0 or ib == 0:
        return None
    if mode == "block16":
        return K.tile_topk(G, keep_count(1.0 - sparsity_ratio, bs * bs), G.dtype)
    means = K.block_stat(mask, bs, L.BLOCK_MEAN)
    keep = K.topk_keep(means, keep_count(1.0 - sparsity_ratio, ob * ib))
    return K.block_fill(keep, torch.empty_like(G), bs, edge_val=1.0)
