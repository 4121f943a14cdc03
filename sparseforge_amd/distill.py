"""Distillation KL of Distill_Model (legacy/sparse_modeling.py:1749-1828) on the HIP kernels.

KL(P_teacher || Q_student) at temperature T over the vocabulary, logits
clamped to +-100; per chunk of token rows (sf_kl_chunk_rows: 2048, 512 or 128
by vocabulary size) a chunk with a NaN log-probability is skipped and a
non-finite chunk sum dropped; the total is scaled by T^2 / tokens and cast to
the student dtype (0 if not finite).  One fused pass reads both logit rows
(sf_kl_forward); the backward re-reads them (sf_kl_backward) and gives the
student gradient g (T / tokens) (q - p) inside the clamp range.  The teacher
takes no gradient (the reference computes it under no_grad).

Difference from the reference: for float32 logits the reference's
`.float().clamp_().mul_()` rewrites the caller's tensors in place; here the
inputs are left unchanged (the loss is the same).
"""
from __future__ import annotations

import torch

from . import _lib as L
from . import profiling as _prof


class _KL(torch.autograd.Function):
    @staticmethod
    def forward(ctx, s2: torch.Tensor, t2: torch.Tensor, temperature: float, out_dtype: torch.dtype):
        dev = L.require_device(s2, t2)
        rows, vocab = s2.shape
        out = torch.empty((), dtype=out_dtype, device=dev)
        lse = torch.empty(rows, 2, dtype=torch.float64, device=dev)
        scale = torch.empty(rows, dtype=torch.float32, device=dev)
        lib = L.lib()
        ws = torch.empty(max(int(lib.sf_kl_workspace_size(rows)), 1), dtype=torch.uint8, device=dev)
        with _prof.region("sf_kl_forward", 2 * s2.numel() * s2.element_size(), "B", dev):
            L.check(lib.sf_kl_forward(L.ptr(s2), L.ptr(t2), L.dtype_code(s2), rows, vocab, float(temperature),
                                      int(lib.sf_kl_chunk_rows(vocab)), L.ptr(out), L.dtype_code(out), L.ptr(lse),
                                      L.ptr(scale), L.ptr(ws), ws.numel(), L.stream(dev)), "sf_kl_forward")
        ctx.save_for_backward(s2, t2, lse, scale)
        ctx.temperature = float(temperature)
        return out

    @staticmethod
    def backward(ctx, g):
        s2, t2, lse, scale = ctx.saved_tensors
        # a Function of its own, so that torch.autograd.grad(..., create_graph=True) (the Hutchinson
        # Hessian-vector product) differentiates the KL gradient as the reference's torch ops are
        gs = _KLGrad.apply(s2, t2, lse, scale, g, ctx.temperature)
        return gs, None, None, None


class _KLGrad(torch.autograd.Function):
    """gs = g * c_r * (q - p) inside the clamp range (sf_kl_backward), differentiable once more.

    With q = softmax(clamp(s) / T) per row, m = [-100 <= s <= 100] and c_r the row scale
    (T / rows, or 0 for a skipped chunk): d gs_i / d s_j = m_i m_j (g c_r / T) q_i (delta_ij - q_j),
    so the vector-Jacobian product with u = ggs * m is
        s_bar_j = m_j (g c_r / T) q_j (u_j - sum_i u_i q_i),
    and d gs / d g = c_r m (q - p) gives g_bar = sum ggs * c_r * m * (q - p).  These run as float32
    device elementwise ops and row sums (they are needed once per Hutchinson probe).  Rows of a dropped
    chunk (c_r = 0) give exact zeros even where their logits are NaN."""

    @staticmethod
    def forward(ctx, s2, t2, lse, scale, g, temperature: float):
        dev = s2.device
        gg = g.detach().contiguous()
        if gg.dtype not in (torch.float32, torch.bfloat16):
            gg = gg.float()
        gs = torch.empty_like(s2)
        rows, vocab = s2.shape
        with _prof.region("sf_kl_backward", 3 * s2.numel() * s2.element_size(), "B", dev):
            L.check(L.lib().sf_kl_backward(L.ptr(s2), L.ptr(t2), L.dtype_code(s2), rows, vocab, float(temperature),
                                           L.ptr(lse), L.ptr(scale), L.ptr(gg), L.dtype_code(gg), L.ptr(gs),
                                           L.stream(dev)), "sf_kl_backward")
        ctx.save_for_backward(s2, t2, lse, scale, g)
        ctx.temperature = float(temperature)
        return gs

    @staticmethod
    def backward(ctx, ggs):
        s2, t2, lse, scale, g = ctx.saved_tensors
        T = ctx.temperature
        s = s2.float()
        # live: inside the clamp range in a chunk the forward kept (row scale > 0).  A dropped chunk may hold
        # NaN logits (that is why it was dropped), and the reference takes it out of the graph, so every
        # term there is selected to 0 rather than multiplied by 0 (0 * NaN would be NaN).
        live = (s >= -100.0) & (s <= 100.0) & (scale > 0)[:, None]
        q = torch.where(live, torch.exp(s.clamp(-100.0, 100.0) / T - lse[:, 0:1].float()), 0.0)
        u = torch.where(live, ggs.float(), 0.0)
        dot = (u * q).sum(dim=1, keepdim=True)
        coef = (g.float() * scale / T)[:, None]
        s_bar = torch.where(live, coef * q * (u - dot), 0.0).to(s2.dtype)
        g_bar = None
        if ctx.needs_input_grad[4]:
            p = torch.where(live, torch.exp(t2.float().clamp(-100.0, 100.0) / T - lse[:, 1:2].float()), 0.0)
            g_bar = (u * (q - p) * scale[:, None]).sum().to(g.dtype).reshape(g.shape)
        return s_bar, None, None, None, g_bar, None


def chunked_kl_loss(student_logits: torch.Tensor, teacher_logits: torch.Tensor, temperature=2) -> torch.Tensor:
    """Distill_Model.kl_loss(student_logits, teacher_logits, temperature) (:1749-1828)."""
    shape = student_logits.shape
    dtype = student_logits.dtype
    s2 = student_logits.reshape(-1, shape[-1])
    t2 = teacher_logits.reshape(-1, shape[-1]).detach()
    if t2.dtype != s2.dtype:
        t2 = t2.to(s2.dtype)
    if s2.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"kl_loss: logits dtype {s2.dtype} (float32 / bfloat16 only)")
    return _KL.apply(s2.contiguous(), t2.contiguous(), float(temperature), dtype)
