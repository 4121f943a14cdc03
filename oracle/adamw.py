"""Oracle of the mask-aware AdamW step (legacy/adamw.py:65-176).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  numpy float32 in the
reference's op order, with the rounding of torch's CPU kernels for each op
(measured on torch 2.10, recorded in the test that pins this module):

  mul by a Python scalar      RN(x * f32(s))
  add(other, alpha=a)         fma(other, f32(a), self)          one rounding
  addcmul(t1, t2, value=v)    fma(RN(f32(v) * t1), t2, self)
  addcdiv(t1, t2, value=v)    RN(self + RN(RN(f32(v) * t1) / t2))
  div by a Python scalar      RN(x / f32(s))
  sqrt                        IEEE sqrt (correctly rounded).  torch's CPU
                              kernel on AVX-512 is not: about 0.6 % of its
                              results are 1 ulp low, so the reference's own
                              CPU outputs differ from this by a few ulp.

Pinned by tests/test_oracle_adamw.py: torch.optim.AdamW(foreach=False) for
decay = 0 / l1 = 0 (the same decoupled-decay formula), the same with the
masked-decay term pre-added to the gradient for decay != 0, the reference's
own outputs (tests/golden/ref_adamw_*.npz) within the fp32 bar, and a
closed form of the L1 term.
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32
F64 = np.float64


def _fma(a, b, c) -> np.ndarray:
    """a * b + c with one rounding to f32 (the product is exact in f64)."""
    return (np.asarray(a, F64) * np.asarray(b, F64) + np.asarray(c, F64)).astype(F32)


def step(p, g, m, v, vmax, mask, step_no: int, lr: float, betas, eps: float, weight_decay: float, decay: float = 0.0,
         l1: float = 0.0, amsgrad: bool = False):
    """One AdamW.step for one f32 parameter; returns (p, m, v, vmax).

    step_no: state['step'] after the increment (:146).  mask: the parameter's
    `mask` attribute or None.  l1 applies to parameters of dim >= 2 with a mask.
    """
    b1, b2 = betas
    p = (np.asarray(p, F32) * F32(1 - lr * weight_decay)).astype(F32)  # :85
    g = np.asarray(g, F32)
    if mask is not None:  # :98-109
        t = (p * (F32(1) - np.asarray(mask, F32)).astype(F32)).astype(F32)
        g = _fma(t, F32(decay), g)
    bc1 = 1 - b1 ** step_no  # :147-148
    bc2 = 1 - b2 ** step_no
    m = (np.asarray(m, F32) * F32(b1)).astype(F32)  # :151
    m = _fma(g, F32(1 - b1), m)
    v = (np.asarray(v, F32) * F32(b2)).astype(F32)  # :152
    v = _fma((F32(1 - b2) * g).astype(F32), g, v)
    vv = v
    if amsgrad:  # :153-157
        vmax = np.maximum(np.asarray(vmax, F32), v)
        vv = vmax
    denom = ((np.sqrt(vv).astype(F32) / F32(math.sqrt(bc2))).astype(F32) + F32(eps)).astype(F32)  # :157-159
    step_size = lr / bc1  # :161
    p = (p + ((F32(-step_size) * m).astype(F32) / denom).astype(F32)).astype(F32)  # :163
    if l1 > 0.0 and mask is not None and p.ndim >= 2:  # :171-174
        lt = ((F32(l1) * np.sign(p)).astype(F32) / denom).astype(F32)
        p = _fma(lt, F32(-lr), p)
    return p, m, v, vmax


def bytes_per_param(masked: bool = True, amsgrad: bool = False, master_copy: bool = True, p_bytes: int = 4,
                    g_bytes: int = 2, s_bytes: int = 4, m_bytes: int = 4) -> int:
    """HBM bytes one fused step moves per parameter (each tensor read / written once)."""
    b = 2 * p_bytes + g_bytes + 2 * 2 * s_bytes
    if amsgrad:
        b += 2 * s_bytes
    if masked:
        b += m_bytes
    if master_copy:
        b += 2
    return b
