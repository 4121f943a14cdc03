"""Oracle of the masked linear + SLoRB forward/backward (K1-K5).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  numpy float32 (or
float64) restatement of

  FusedMaskedLinearSTE.forward   legacy/sparse_modeling.py:72-93
      w = W * mask_cast (* scale_factor);  y = x w^T + b
  FusedMaskedLinearSTE.backward  legacy/sparse_modeling.py:96-132
      dx = dy (W * mask)           (no scale factor: :113-115)
      dW = dy^T x                  (straight-through, unmasked: :120)
           + decay * W * [mask < 0.5]   (only when decay != 0: :123-125)
      db = sum_t dy                (:127-129)
  SLoRB bypass                   legacy/sparse_modeling.py:790-794
      y += (x P^T) S^T  ->  dz = dy S,  dx += dz P,  dP = dz^T x,  dS = dy^T z
  effective mask                 legacy/sparse_modeling.py:759-771
      E = soft (hx >= 1 - 1e-6)  |  hx * soft + (1 - hx) * hard(soft)

Pinned by tests/test_oracle_linear.py against the reference's own outputs
(tests/golden/ref_linear_slorb_f32.npz, written by running
FusedMaskedLinearSTE + SLoRB) and against torch.autograd on the dense
equivalent, which fixes every transpose and the STE convention.
"""
from __future__ import annotations

import numpy as np

from .masks import hard_mask_from_soft


def effective_mask(soft: np.ndarray, hx: float, hard_type: str = "nm_2_4", N: int = 2, M: int = 4) -> np.ndarray:
    """E of SparseLinear.forward for a non-finalized layer (:759-771)."""
    soft = np.asarray(soft, dtype=np.float32)
    if hx >= 1.0 - 1e-6:
        return soft
    hard = hard_mask_from_soft(soft, hard_type, N, M)
    return (np.float32(hx) * soft + np.float32(1.0 - hx) * hard).astype(np.float32)


def weight_scale(hx: float, target: float) -> float:
    """1 + (1 - hx) (target - 1) of weight_scaling (:779-784)."""
    return 1.0 + (1.0 - hx) * (target - 1.0)


def forward(x, W, E, b=None, scale: float = 1.0, P=None, S=None, dtype=np.float32):
    """y [T, out] = x (W E s)^T + b + (x P^T) S^T  for x [T, in]."""
    x = np.asarray(x, dtype=dtype)
    w = np.asarray(W, dtype=dtype) * np.asarray(E, dtype=dtype)
    if scale != 1.0:
        w = w * dtype(scale)
    y = x @ w.T
    if b is not None:
        y = y + np.asarray(b, dtype=dtype)
    if P is not None:
        y = y + (x @ np.asarray(P, dtype=dtype).T) @ np.asarray(S, dtype=dtype).T
    return y


def backward(x, W, E, gy, has_bias: bool = True, P=None, S=None, decay: float = 0.0, dtype=np.float32) -> dict:
    """Gradients of the STE backward (:96-132) and of the SLoRB pair."""
    x = np.asarray(x, dtype=dtype)
    W = np.asarray(W, dtype=dtype)
    E = np.asarray(E, dtype=dtype)
    gy = np.asarray(gy, dtype=dtype)
    out = {"dx": gy @ (W * E), "dW": gy.T @ x}
    if decay != 0.0:
        out["dW"] = out["dW"] + dtype(decay) * W * (E < 0.5).astype(dtype)
    out["db"] = gy.sum(0) if has_bias else None
    if P is not None:
        P = np.asarray(P, dtype=dtype)
        S = np.asarray(S, dtype=dtype)
        z = x @ P.T
        dz = gy @ S
        out["dx"] = out["dx"] + dz @ P
        out["dP"] = dz.T @ x
        out["dS"] = gy.T @ z
    return out


def flops_fwd_bwd(tokens: int, in_f: int, out_f: int, rank: int = 0) -> int:
    """Algorithmic FLOPs of one fwd+bwd: 6 T in out + 6 T r (in + out)."""
    return 6 * tokens * in_f * out_f + 6 * tokens * rank * (in_f + out_f)
