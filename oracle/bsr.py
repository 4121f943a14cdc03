"""Oracle of the block-sparse-16 format and products (legacy/triton_block_sparse.py).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

* convert: convert_to_block_sparse (:46-103): W * mask in the promoted dtype,
  a block kept iff sum(|block|) > 0 (so a block holding a NaN is dropped),
  CSR over block rows with ascending column indices, and a single zero
  block (with an empty index) when nothing is kept.
* to_dense: the block layout expanded back (the reference's _torch_forward
  rebuild, :435-462).
* block_map: [nbr, nbc] block indices, -1 where pruned.
* forward / input_grad / sddmm_grad: y = x W^T, dx = dy W, and dW restricted
  to the kept blocks, from the dense expansion.

Pinned by tests/test_oracle_bsr.py against the reference's own output
(tests/golden/ref_bsr_basic_f32.npz) and a brute-force per-block scan.
"""
from __future__ import annotations

import numpy as np


def convert(W: np.ndarray, mask: np.ndarray, bs: int = 16):
    """(blocks [nnz, bs, bs], row_ptr int32 [nbr + 1], col_idx int32 [nnz])."""
    W = np.asarray(W, np.float32)
    out_f, in_f = W.shape
    assert out_f % bs == 0 and in_f % bs == 0
    nbr, nbc = out_f // bs, in_f // bs
    sw = (W * np.asarray(mask, np.float32)).astype(np.float32)
    blocked = sw.reshape(nbr, bs, nbc, bs).transpose(0, 2, 1, 3)
    with np.errstate(invalid="ignore"):
        norms = np.abs(blocked).sum(axis=(-1, -2))
    blocks, row_ptr, col_idx = [], [0], []
    for r in range(nbr):
        for c in np.nonzero(norms[r] > 0)[0]:
            blocks.append(blocked[r, c])
            col_idx.append(int(c))
        row_ptr.append(len(blocks))
    if not blocks:
        arr = np.zeros((1, bs, bs), np.float32)
    else:
        arr = np.stack(blocks).astype(np.float32)
    return arr, np.asarray(row_ptr, np.int32), np.asarray(col_idx, np.int32)


def block_map(row_ptr: np.ndarray, col_idx: np.ndarray, nbr: int, nbc: int) -> np.ndarray:
    m = np.full((nbr, nbc), -1, np.int32)
    for r in range(nbr):
        for k in range(int(row_ptr[r]), int(row_ptr[r + 1])):
            m[r, int(col_idx[k])] = k
    return m


def to_dense(blocks: np.ndarray, row_ptr: np.ndarray, col_idx: np.ndarray, out_f: int, in_f: int,
             bs: int = 16) -> np.ndarray:
    W = np.zeros((out_f, in_f), np.float32)
    for r in range(out_f // bs):
        for k in range(int(row_ptr[r]), int(row_ptr[r + 1])):
            c = int(col_idx[k])
            W[r * bs:(r + 1) * bs, c * bs:(c + 1) * bs] = blocks[k]
    return W


def forward(x, blocks, row_ptr, col_idx, out_f, in_f, bs=16):
    return np.asarray(x, np.float64) @ to_dense(blocks, row_ptr, col_idx, out_f, in_f, bs).astype(np.float64).T


def input_grad(gy, blocks, row_ptr, col_idx, out_f, in_f, bs=16):
    return np.asarray(gy, np.float64) @ to_dense(blocks, row_ptr, col_idx, out_f, in_f, bs).astype(np.float64)


def sddmm_grad(gy, x, row_ptr, col_idx, bs=16):
    """dW at the kept blocks: blocks [nnz, bs, bs] of gy^T x."""
    full = np.asarray(gy, np.float64).T @ np.asarray(x, np.float64)
    out = []
    for r in range(len(row_ptr) - 1):
        for k in range(int(row_ptr[r]), int(row_ptr[r + 1])):
            c = int(col_idx[k])
            out.append(full[r * bs:(r + 1) * bs, c * bs:(c + 1) * bs])
    return np.stack(out) if out else np.zeros((0, bs, bs))


def flops(tokens: int, nnz: int, bs: int = 16) -> int:
    """Algorithmic FLOPs of one block-sparse product: 2 T nnz bs^2 (kept blocks only)."""
    return 2 * tokens * nnz * bs * bs
