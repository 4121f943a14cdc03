"""Oracle of the 2:4 packed weight layout (sf_pack_2to4 / sf_unpack_2to4).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  The reference stores a
finalized weight densely: W * M_hard (legacy/main_llama.py:2499-2568) and runs
F.linear(x, W * M_hard) (legacy/eval_wiki_ppl.py:548-651).  The packed form
has no reference counterpart; it is pinned by the round trip
unpack(pack(W, M)) == W * M (bit-exact for 2:4 masks) and by the product
x . unpack(p)^T against the dense finalized forward.

Layout: vals [out, in / 2] bf16, the two kept values of each group of 4 in
column order (groups keeping fewer are padded with zeros at their lowest
unused columns); idx u32 [out / 32][in / 64][2][32]: word (rb, q, h, r) holds
the 2-bit in-group columns of the 8 kept values of row rb * 32 + r, columns
[64 q + 16 h, +16) in bits 0..15 and [64 q + 32 + 16 h, +16) in bits 16..31.
pack() / unpack() keep vals in that row order; the device stores the same
values in the sparse MFMA's fragment order, tile_vals() (pinned by the
round trip through the device pack and unpack).
"""
from __future__ import annotations

import numpy as np

from .numerics import round_bf16


def pack(W: np.ndarray, mask: np.ndarray):
    """(vals float32 [out, in/2] holding bf16 values, idx uint32 [out/32, in/64, 2, 32], bad group count)."""
    W = np.asarray(W, np.float32)
    mask = np.asarray(mask, np.float32)
    out_f, in_f = W.shape
    assert out_f % 32 == 0 and in_f % 64 == 0
    g = out_f * in_f // 4
    keep = (mask != 0).reshape(g, 4)
    prod = (W * mask).astype(np.float32).reshape(g, 4)
    bad = int((keep.sum(1) > 2).sum())
    pos = np.zeros((g, 2), np.int64)
    val = np.zeros((g, 2), np.float32)
    for gi in range(g):
        cols = [c for c in range(4) if keep[gi, c]][:2]
        vs = [prod[gi, c] for c in cols]
        for c in range(4):
            if len(cols) == 2:
                break
            if c not in cols:
                cols.append(c)
                vs.append(np.float32(0.0))
        order = np.argsort(cols, kind="stable")
        pos[gi] = np.array(cols)[order]
        val[gi] = np.array(vs, np.float32)[order]
    vals = round_bf16(val).reshape(out_f, in_f // 2)
    # 16-bit words per (row, 16-column block): value j of the block at bits 2j
    pos = pos.reshape(out_f, in_f // 16, 8)
    w16 = (pos << (2 * np.arange(8))).sum(-1).astype(np.uint32)  # [out, in/16]
    w16 = w16.reshape(out_f // 32, 32, in_f // 64, 4)  # rb, r, q, sub
    idx = np.zeros((out_f // 32, in_f // 64, 2, 32), np.uint32)
    for sub in range(4):
        h, half = sub & 1, sub >> 1
        idx[:, :, h, :] |= (w16[:, :, :, sub].transpose(0, 2, 1) << (16 * half)).astype(np.uint32)
    return vals, idx, bad


def unpack(vals: np.ndarray, idx: np.ndarray, out_f: int, in_f: int) -> np.ndarray:
    W = np.zeros((out_f, in_f), np.float32)
    v = np.asarray(vals, np.float32).reshape(out_f, in_f // 16, 8)
    ix = np.asarray(idx, np.uint32).reshape(out_f // 32, in_f // 64, 2, 32)
    for sub in range(4):
        h, half = sub & 1, sub >> 1
        w = ((ix[:, :, h, :] >> (16 * half)) & 0xFFFF).transpose(0, 2, 1).reshape(out_f, in_f // 64)
        for j in range(8):
            p = ((w >> (2 * j)) & 3).astype(np.int64)
            col = (np.arange(in_f // 64)[None, :] * 64 + sub * 16 + (j // 2) * 4) + p
            rows = np.repeat(np.arange(out_f)[:, None], in_f // 64, axis=1)
            np.add.at(W, (rows, col), v[:, np.arange(in_f // 64) * 4 + sub, j])
    return W


def tile_vals(vals: np.ndarray) -> np.ndarray:
    """vals [out, in / 2] in row order -> the device order (same shape, flattened): the 8 values of
    16-column chunk 4 q + 2 kk + h of row 32 rb + r at [rb][q][kk][h * 32 + r][8]."""
    vals = np.asarray(vals)
    out_f, half = vals.shape
    nk = half // 32
    v = vals.reshape(out_f // 32, 32, nk, 2, 2, 8)  # rb, r, q, kk, h, value
    return np.ascontiguousarray(v.transpose(0, 2, 3, 4, 1, 5)).reshape(out_f, half)


def untile_vals(tiled: np.ndarray) -> np.ndarray:
    """The inverse of tile_vals."""
    tiled = np.asarray(tiled)
    out_f, half = tiled.shape
    nk = half // 32
    v = tiled.reshape(out_f // 32, nk, 2, 2, 32, 8)  # rb, q, kk, h, r, value
    return np.ascontiguousarray(v.transpose(0, 4, 1, 2, 3, 5)).reshape(out_f, half)
