"""Distillation KL of Distill_Model (legacy/sparse_modeling.py:1749-1828).

KL(P_teacher || Q_student) at temperature T over the vocabulary, logits
clamped to +-100, computed in float32 chunks of tokens; a chunk whose
log-probabilities contain NaN is skipped, a non-finite chunk sum is dropped,
and the total is scaled by T^2 / num_tokens.  This wrapper sits at the edge
of the hot path (after the student forward) and uses torch's device ops.
"""
from __future__ import annotations

import torch
from torch.nn import functional as F


def chunked_kl_loss(student_logits: torch.Tensor, teacher_logits: torch.Tensor, temperature=2) -> torch.Tensor:
    shape = student_logits.shape
    device, dtype = student_logits.device, student_logits.dtype
    s_flat = student_logits.reshape(-1, shape[-1])
    t_flat = teacher_logits.reshape(-1, shape[-1])
    n_tok, vocab = s_flat.shape
    chunk = 128 if vocab > 100000 else (512 if vocab > 50000 else 2048)
    inv_t = 1.0 / temperature
    total = torch.tensor(0.0, device=device, dtype=torch.float32)
    for i in range(0, n_tok, chunk):
        j = min(i + chunk, n_tok)
        s_lp = F.log_softmax(s_flat[i:j].float().clamp(-100.0, 100.0) * inv_t, dim=-1)
        t_lp = F.log_softmax(t_flat[i:j].float().clamp(-100.0, 100.0) * inv_t, dim=-1)
        if torch.isnan(s_lp).any() or torch.isnan(t_lp).any():
            continue
        c = ((t_lp - s_lp) * t_lp.exp()).sum()
        if torch.isfinite(c):
            total = total + c
    kl = (total * (temperature ** 2) / n_tok).to(dtype)
    if not torch.isfinite(kl):
        return torch.tensor(0.0, device=device, dtype=dtype)
    return kl
