"""Oracle of one sparse retraining step — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

A float64 CPU restatement of the step of legacy/main_llama.py:1996-2211 on
the LLaMA-architecture decoder of sparseforge_amd/llama.py, for the small
shapes the end-to-end GPU test runs.  The model's gradients and the
Hutchinson double backward come from torch.autograd on the CPU in float64;
every SparseForge-specific piece is one of the pinned oracle functions:

  masked linear   the straight-through product of linear.py (forward
                  x (W E)^T, backward dx = gy (W E), dW = gy^T x; written as
                  an autograd Function whose backward is differentiable ops,
                  as the reference's FusedMaskedLinearSTE.backward is,
                  legacy/sparse_modeling.py:96-132) plus the SLoRB pair
                  (x P^T) S^T (:790-794); E from linear.effective_mask
  distillation    distill.py's KL (:1749-1828) as differentiable torch ops
  Hutchinson      hutchinson.rademacher probes (the device's counter RNG),
                  hvp by double backward, hutchinson.update's f32 EMA
                  (legacy/utils.py:714-869)
  penalties       mid_penalty / sparsity_penalty of unstructured masks
                  (legacy/utils.py:876-1025): constants added to the loss
  clipping        torch.nn.utils.clip_grad_norm_'s formula
  AdamW           adamw.step per parameter (legacy/adamw.py:65-176)
  mask update     masks.layer_update_mask per SparseLinear
                  (legacy/sparse_modeling.py:1242-1666)

The stock pieces (RMSNorm, rotary embedding, causal softmax attention, SwiGLU,
cross-entropy) restate HuggingFace's LlamaForCausalLM, the model the reference
retrains (legacy/model_llama.py:39-55), in float64 except where that model
itself computes in float32 whatever its dtype (the rotary tables, RMSNorm's
normalisation, the attention softmax); tests/test_llama_reference_model.py
pins this forward against transformers' own LlamaForCausalLM in float64.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from . import adamw as oa
from . import hutchinson as oh
from . import linear as ol
from . import masks as om

F64 = torch.float64
LINEARS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
           "mlp.up_proj", "mlp.down_proj")


class _STE(torch.autograd.Function):
    """x (W E)^T with the straight-through backward; the backward is differentiable ops."""

    @staticmethod
    def forward(ctx, x, W, E):
        ctx.save_for_backward(x, W, E)
        return x @ (W * E).t()

    @staticmethod
    def backward(ctx, gy):
        x, W, E = ctx.saved_tensors
        return gy @ (W * E), gy.t() @ x, None


def rmsnorm(x, w, eps):
    """LlamaRMSNorm: the normalisation in float32 whatever the activations' dtype, then the weight."""
    xf = x.to(torch.float32)
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(x.dtype)


def rope(seq, d, theta):
    """cos, sin of HuggingFace's LlamaRotaryEmbedding (the reference's model): inverse frequencies,
    angles, cos and sin in float32, then widened (the module casts them to the activations' dtype)."""
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    ang = torch.arange(seq, dtype=torch.float32)[:, None] * inv[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().to(F64), ang.sin().to(F64)


def _rot(x, cos, sin):
    h = x.shape[-1] // 2
    return x * cos + torch.cat([-x[..., h:], x[..., :h]], dim=-1) * sin


def attention(q, k, v, cos, sin):
    """Eager attention: scores (q k^T) * D^-0.5, causal mask, softmax in float32 cast back, p v."""
    B, S, H, D = q.shape
    q, k, v = (_rot(q.transpose(1, 2), cos, sin), _rot(k.transpose(1, 2), cos, sin), v.transpose(1, 2))
    s = (q @ k.transpose(-2, -1)) * (D ** -0.5)
    s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    return (torch.softmax(s, -1, dtype=torch.float32).to(q.dtype) @ v).transpose(1, 2).reshape(B, S, H * D)


def kl_loss(s, t, T=2.0):
    """Distill_Model.kl_loss in differentiable float64 ops (chunked sum, NaN chunks skipped)."""
    V = s.shape[-1]
    s2 = s.reshape(-1, V).clamp(-100, 100) / T
    t2 = t.reshape(-1, V).clamp(-100, 100) / T
    logq, logp = torch.log_softmax(s2, -1), torch.log_softmax(t2, -1)
    rows = s2.shape[0]
    step = 2048 if V <= 50000 else (512 if V <= 100000 else 128)
    total = s2.new_zeros(())
    for c in range(0, rows, step):
        lq, lp = logq[c:c + step], logp[c:c + step]
        if torch.isnan(lq).any() or torch.isnan(lp).any():
            continue
        part = (lp.exp() * (lp - lq)).sum()
        if torch.isfinite(part):
            total = total + part
    return total * (T * T) / rows


def forward(P, E, shape, idx, student: bool, slorb: bool):
    """Logits of the student (masked linears, effective masks E by module name) or dense teacher."""
    cos, sin = rope(idx.shape[1], shape.head_dim, shape.rope_theta)
    h = P["embed_tokens.weight"][idx]

    def lin(x, name):
        x2 = x.reshape(-1, x.shape[-1])
        if not student:
            y = x2 @ P[name + ".weight"].t()
        else:
            y = _STE.apply(x2, P[name + ".weight"], E[name])
            if slorb:
                y = y + (x2 @ P[name + ".x_proj"].t()) @ P[name + ".SLoRB_Weight"].t()
        return y.reshape(*x.shape[:-1], -1)

    for li in range(shape.num_hidden_layers):
        pre = f"layers.{li}."
        n = rmsnorm(h, P[pre + "input_layernorm.weight"], shape.rms_norm_eps)
        B, S, _ = n.shape
        q = lin(n, pre + "self_attn.q_proj").view(B, S, shape.num_attention_heads, -1)
        k = lin(n, pre + "self_attn.k_proj").view(B, S, shape.num_attention_heads, -1)
        v = lin(n, pre + "self_attn.v_proj").view(B, S, shape.num_attention_heads, -1)
        h = h + lin(attention(q, k, v, cos, sin), pre + "self_attn.o_proj")
        n = rmsnorm(h, P[pre + "post_attention_layernorm.weight"], shape.rms_norm_eps)
        h = h + lin(F.silu(lin(n, pre + "mlp.gate_proj")) * lin(n, pre + "mlp.up_proj"), pre + "mlp.down_proj")
    return rmsnorm(h, P["norm.weight"], shape.rms_norm_eps) @ P["lm_head.weight"].t()


def sparse_names(shape):
    return [f"layers.{li}.{n}" for li in range(shape.num_hidden_layers) for n in LINEARS]


def step(state: dict, teacher: dict, shape, cfg: dict, step_cfg: dict, iter_num: int, batches, seed0: int) -> dict:
    """One retraining step.

    state: numpy f32 arrays by parameter name (student parameters, plus per SparseLinear
    `<name>.mask` and `<name>.hessian_diag`, and AdamW moments `<param>.exp_avg` /
    `<param>.exp_avg_sq` with `<param>.step`), hardening `<name>.hx`; teacher: parameters.
    cfg: the SparseLinear config (oracle.masks.full_config); step_cfg: RetrainConfig fields.
    batches: list of (X, Y) int64 arrays; seed0: seed of the first Hutchinson probe (the
    probes take seed0, seed0 + 1, ... in module order).  Returns the new state plus the
    intermediate quantities the test compares (loss, clipped grads, hessian after the probe).
    """
    names = sparse_names(shape)
    slorb = bool(cfg["SLoRB"])
    trainable = [k for k in state if _is_param(k, names, slorb, cfg)]
    P = {k: torch.tensor(state[k], dtype=F64, requires_grad=k in trainable) for k in state
         if not _is_aux(k)}
    T_ = {k: torch.tensor(v, dtype=F64) for k, v in teacher.items()}
    E = {}
    for n in names:
        hx = float(state[n + ".hx"])
        soft = state[n + ".mask"]
        E[n] = torch.tensor(ol.effective_mask(soft, hx, om.effective_hard_type(cfg)) if hx < 1.0 - 1e-6 else soft,
                            dtype=F64)
    warm = 2000 if step_cfg["mask_penalty_mode"] in ("block_sparse16", "block_sparse32", "block16") else 500
    lam = step_cfg["lambda_mid_max"] * (iter_num / warm) if iter_num < warm else step_cfg["lambda_mid_max"]
    masks = [state[n + ".mask"].astype(np.float64) for n in names]
    mid = lam * sum(float((m * (1 - m)).sum()) for m in masks) / sum(m.size for m in masks) if lam > 0 else 0.0
    sp = 0.0
    if step_cfg["sparsity_alpha"]:
        frac = sum(int((m < 0.5).sum()) for m in masks) / sum(m.size for m in masks)
        sp = step_cfg["sparsity_alpha"] * (frac - step_cfg["sparsity_ratio"]) ** 2
    GA = step_cfg["grad_accum"]
    out = {"loss": 0.0}
    H = {n: state[n + ".hessian_diag"].copy() for n in names}
    for micro, (X, Y) in enumerate(batches):
        X, Y = torch.as_tensor(X), torch.as_tensor(Y)
        logits = forward(P, E, shape, X, True, slorb)
        with torch.no_grad():
            t_logits = forward(T_, None, shape, X, False, False)
        task = F.cross_entropy(logits.reshape(-1, logits.shape[-1]), Y.reshape(-1), ignore_index=-1)
        loss = step_cfg["hardness_task"] * task + step_cfg["hardness_kldiv"] * kl_loss(logits, t_logits)
        loss = (loss + mid + sp) / GA
        if micro == GA - 1 and step_cfg["hutchinson"]:
            Ws = [P[n + ".weight"] for n in names]
            grads = torch.autograd.grad(loss, Ws, create_graph=True)
            vs = [torch.tensor(oh.rademacher(seed0 + j, W.numel()).reshape(W.shape), dtype=F64)
                  for j, W in enumerate(Ws)]
            dot = sum((g * v).sum() for g, v in zip(grads, vs))
            hvps = torch.autograd.grad(dot, Ws, retain_graph=True)
            for n, hvp, v in zip(names, hvps, vs):
                H[n] = oh.update(H[n], hvp.numpy().astype(np.float32), v.numpy().astype(np.float32),
                                 float(cfg["beta"]))
                out[n + ".hvp"] = hvp.numpy()
        loss.backward()
        out["loss"] += float(loss.detach())
    grads = {k: P[k].grad.numpy().copy() for k in trainable}
    if step_cfg["grad_clip"]:
        norm = math.sqrt(sum(float((g.astype(np.float64) ** 2).sum()) for g in grads.values()))
        coef = min(step_cfg["grad_clip"] / (norm + 1e-6), 1.0)
        grads = {k: g * coef for k, g in grads.items()}
        out["grad_norm"] = norm
    out["grads"] = grads
    out["hessian"] = H
    new = dict(state)
    for n in names:
        new[n + ".hessian_diag"] = H[n]
    lr, (b1, b2), eps, wd = step_cfg["lr"], step_cfg["betas"], step_cfg["eps"], step_cfg["weight_decay"]
    for k in trainable:
        p = state[k]
        mask = state[k[: -len(".weight")] + ".mask"] if (k.endswith(".weight") and k[: -len(".weight")] in names) \
            else None
        st = int(state.get(k + ".step", 0)) + 1
        m0 = state.get(k + ".exp_avg", np.zeros_like(p))
        v0 = state.get(k + ".exp_avg_sq", np.zeros_like(p))
        p1, m1, v1, _ = oa.step(p, grads[k].astype(np.float32), m0, v0, None, mask, st, lr, (b1, b2), eps,
                                wd if p.ndim >= 2 else 0.0, decay=step_cfg["decay"] if mask is not None else 0.0)
        new[k], new[k + ".exp_avg"], new[k + ".exp_avg_sq"], new[k + ".step"] = p1, m1, v1, st
    flips = {}
    for n in names:
        res = om.layer_update_mask(cfg, iter_num, new[n + ".weight"], new[n + ".hessian_diag"], state[n + ".mask"],
                                   None, None, lam)
        if res is not None:
            new[n + ".mask"], _fr, flips[n], new[n + ".hx"] = res
    out["flips"] = flips
    out["state"] = new
    out["lambda_mid"] = lam
    return out


def _is_aux(k: str) -> bool:
    return k.endswith((".mask", ".hessian_diag", ".exp_avg", ".exp_avg_sq", ".step", ".hx"))


def _is_param(k: str, names, slorb: bool, cfg) -> bool:
    if _is_aux(k):
        return False
    if k.endswith(".x_proj"):
        return bool(cfg["trainable_projection"])
    return True
