"""Oracle of the Hutchinson Hessian-diagonal update (legacy/utils.py:710-869).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

* splitmix64 / rademacher: the counter-based probe the HIP kernels use in
  place of torch.randint (SplitMix64: G. Steele, D. Lea, C. Flood, OOPSLA
  2014; output k of the stream seeded with s is mix64(s + (k + 1) * golden)).
  Pinned by the published first outputs of the stream seeded with 1234567.
* update: H <- beta H + (1 - beta) clamp(hvp v, 0) in the reference's op
  order (:806-868), pinned by the reference's own outputs
  (tests/golden/ref_hutch_quadratic_f32.npz) given its probes.
* quadratic_hvp: for L = 1/2 ||x (W.M)^T - y||^2 under the straight-through
  backward, hvp = v (x^T x) row-wise: the second derivative of the masked
  forward is taken through the same straight-through backward, so the mask
  drops out (checked against torch.autograd and the reference's outputs);
  the expectation of hvp * v over v is diag(x^T x) in every row.
"""
from __future__ import annotations

import numpy as np

_M64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15


def splitmix64(seed: int, k: np.ndarray) -> np.ndarray:
    """Output k (0-based) of the SplitMix64 stream seeded with `seed`, as uint64."""
    k = np.asarray(k, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & _M64) + (k + np.uint64(1)) * np.uint64(GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def rademacher(seed: int, n: int) -> np.ndarray:
    """v_i = +1 if bit (i % 64) of splitmix64(seed, i // 64) is set, else -1 (float32)."""
    i = np.arange(n, dtype=np.uint64)
    h = splitmix64(seed, i >> np.uint64(6))
    bit = (h >> (i & np.uint64(63))) & np.uint64(1)
    return np.where(bit == 1, np.float32(1.0), np.float32(-1.0)).astype(np.float32)


def update(H: np.ndarray, hvp: np.ndarray, v: np.ndarray, beta: float) -> np.ndarray:
    """hessian_diag.mul_(beta).add_(clamp(hvp * v, min=0), alpha=1 - beta) in f32 (:806-868)."""
    est = (np.asarray(hvp, np.float32) * np.asarray(v, np.float32)).astype(np.float32)
    est = np.where(est < 0, np.float32(0), est)
    h = (np.asarray(H, np.float32) * np.float32(beta)).astype(np.float32)
    return (est.astype(np.float64) * np.float32(1 - beta) + h.astype(np.float64)).astype(np.float32)


def quadratic_hvp(x: np.ndarray, v: np.ndarray, E: np.ndarray | None = None, decay: float = 0.0) -> np.ndarray:
    """HVP of 1/2 ||x (W.M)^T - y||^2 w.r.t. W along v under the STE backward: v (x^T x) (the mask drops out).

    With the SR-STE term (decay != 0, legacy/sparse_modeling.py:123-125) the weight gradient also
    holds decay * W * [E < 0.5], whose derivative along v adds decay * v * [E < 0.5]."""
    xtx = np.asarray(x, np.float64).T @ np.asarray(x, np.float64)
    hvp = np.asarray(v, np.float64) @ xtx
    if decay != 0.0:
        hvp = hvp + decay * np.asarray(v, np.float64) * (np.asarray(E, np.float64) < 0.5)
    return hvp
