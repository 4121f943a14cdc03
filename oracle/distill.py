"""Oracle of the distillation KL: Distill_Model.kl_loss (legacy/sparse_modeling.py:1749-1828).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  numpy: the logits are
clamped to +-100 and scaled by 1/T in float32 as the reference does
(:1788-1796); log-softmax, the per-chunk sums and the total run in float64.
Chunks of `chunk_rows(vocab)` token rows whose log-probabilities hold a NaN are
skipped and a non-finite chunk sum is dropped (:1800-1816); the loss is
(f32(total) * T^2) / tokens in float32 (:1821), 0 if not finite (:1825-1826).
"""
from __future__ import annotations

import numpy as np


def chunk_rows(vocab: int) -> int:
    """:1772-1777"""
    return 128 if vocab > 100000 else (512 if vocab > 50000 else 2048)


def _scaled(x: np.ndarray, temperature: float) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    return (np.clip(x, np.float32(-100.0), np.float32(100.0)) * np.float32(1.0 / temperature)).astype(np.float32)


def _log_softmax64(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float64)
    m = np.max(x, axis=-1, keepdims=True)
    return x - m - np.log(np.exp(x - m).sum(-1, keepdims=True))


def kl_parts(s: np.ndarray, t: np.ndarray, temperature: float = 2.0):
    """(loss as float32, per-row kept flags): the reference's chunk loop in float64."""
    v = s.shape[-1]
    s2 = np.asarray(s, np.float32).reshape(-1, v)
    t2 = np.asarray(t, np.float32).reshape(-1, v)
    n = s2.shape[0]
    c = chunk_rows(v)
    total = 0.0
    kept = np.zeros(n, dtype=bool)
    for i in range(0, n, c):
        j = min(i + c, n)
        nan = np.isnan(s2[i:j]).any() or np.isnan(t2[i:j]).any()  # a NaN logit makes its row's log-softmax NaN
        if nan:
            continue
        ls = _log_softmax64(_scaled(s2[i:j], temperature))
        lt = _log_softmax64(_scaled(t2[i:j], temperature))
        chunk = float((np.exp(lt) * (lt - ls)).sum())
        if np.isfinite(chunk):
            total += chunk
            kept[i:j] = True
    kl = np.float32(np.float32(total) * np.float32(temperature ** 2)) / np.float32(n)
    return (np.float32(kl) if np.isfinite(kl) else np.float32(0.0)), kept


def kl_loss(s: np.ndarray, t: np.ndarray, temperature: float = 2.0) -> np.float32:
    return kl_parts(s, t, temperature)[0]


def kl_grad(s: np.ndarray, t: np.ndarray, temperature: float = 2.0, g: float = 1.0) -> np.ndarray:
    """d loss / d student logits (float64): g (T / tokens) (q - p) inside the clamp range, 0 in skipped chunks."""
    v = s.shape[-1]
    s2 = np.asarray(s, np.float32).reshape(-1, v)
    t2 = np.asarray(t, np.float32).reshape(-1, v)
    n = s2.shape[0]
    loss, kept = kl_parts(s, t, temperature)
    q = np.exp(_log_softmax64(_scaled(s2, temperature)))
    p = np.exp(_log_softmax64(_scaled(t2, temperature)))
    inside = (s2 >= -100.0) & (s2 <= 100.0)
    scale = g * temperature / n if np.isfinite(loss) else 0.0
    gr = scale * (q - p) * inside * kept[:, None]
    gr[~kept] = 0.0
    return gr.reshape(np.shape(s))
