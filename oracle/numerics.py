"""Float helpers of the oracle: bf16 rounding and torch-ordered keys (test infrastructure only)."""
from __future__ import annotations

import numpy as np

F32 = "f32"
BF16 = "bf16"


def round_bf16(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), returned as float32.

    Same rounding as torch's ``.to(torch.bfloat16)`` on the CPU (c10/util/BFloat16.h
    round_to_nearest_even); NaN stays NaN.
    """
    a = np.asarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), np.float32(np.nan), out).astype(np.float32)


def rnd(x, dtype: str) -> np.ndarray:
    """Round to the storage dtype of a torch op's result."""
    a = np.asarray(x, dtype=np.float32)
    return round_bf16(a) if dtype == BF16 else a


def promote(a: str, b: str) -> str:
    return F32 if F32 in (a, b) else BF16


def ordered_keys(x) -> np.ndarray:
    """uint32 keys with torch's comparison order: NaN largest (all NaN equal), -0 == +0."""
    a = np.asarray(x, dtype=np.float32)
    u = a.view(np.uint32).copy()
    u[(u & 0x7FFFFFFF) == 0] = 0
    k = np.where(u & 0x80000000, ~u, u | 0x80000000).astype(np.uint32)
    k[np.isnan(a)] = 0xFFFFFFFF
    return k


def sigmoid_f32(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (np.float32(1.0) / (np.float32(1.0) + np.exp(-x))).astype(np.float32)
