"""GLU gate/up joint mask update (legacy/utils.py:363-643) on the HIP kernels.

gate_proj and up_proj outputs are multiplied elementwise, so the reference
prunes both with ONE target: G comes from the summed importance scores of the
pair and is EMA'd into both masks.  Device flow (three reads of the joint
score, one of each mask):

  sf_joint_scores      S = score(gate) + score(up)                (:415-420)
  sf_score_stats       mean / population std of S                 (:541-545)
  sf_tau_quantile      unstructured tau over a sample of z(S)     (:553-556)
  sf_glu_update_masks  G (gate mask / frozen flags), penalty against the
                       gate mask, binarisation, EMA of both masks,
                       per-layer flip counts                      (:422-479)
"""
from __future__ import annotations

import warnings

import torch

from . import _lib as L
from . import kernels as K


def _tag(dt: torch.dtype) -> int:
    return L.DT_BF16 if dt == torch.bfloat16 else L.DT_F32


def _joint_params(gate, step: int, rows: int, cols: int, mask_dtype: torch.dtype, has_frozen: bool,
                  lambda_mid: float) -> L.MaskParams:
    """Host scalars of _compute_joint_gate_target (:536-613) and the update half (:422-479)."""
    p = L.MaskParams()
    p.rows, p.cols = rows, cols
    p.metric = L.METRIC["hessian"]  # the score is S itself
    N, M = int(gate.N), int(gate.M)
    if gate.mask_type == "structured":
        assert cols % M == 0, f"in_features ({cols}) must be divisible by M ({M})."
        p.gate = L.GATE_STRUCTURED_EXACT if getattr(gate.cfg, "structured_exact", False) else L.GATE_STRUCTURED
    else:  # unstructured, and the reference's default branch
        p.gate = L.GATE_UNSTRUCTURED
    p.n_keep, p.m_group = N, M
    p.score_dtype = _tag(mask_dtype)  # z and G are held in the mask dtype (:545)
    p.temperature = gate._temperature(step)
    p.eps_metric = 1e-8
    p.movement_temp = 1.0
    p.beta_struct = gate._beta_structural(step) if cols >= M else 0.0
    p.has_frozen = int(has_frozen)
    # block hard types count flips from whole-tensor projections after the pass
    kind, hn, hm = (L.HARD_THRESHOLD, 2, 4) if gate._is_block_hard() else gate._hard_kind()
    p.hard_kind, p.hard_n, p.hard_m = kind, hn, hm
    p.penalty, p.penalty_coef = L.PENALTY_NONE, 0.0
    lam = float(lambda_mid) if lambda_mid is not None else 0.0
    if lam != 0.0:
        mode = str(getattr(gate.cfg, "mask_penalty_mode", "mid") or "mid")
        if mode == "structured_topn" and cols % M != 0:
            mode = "mid"
        # other modes leave G as it is (their clamp to [0, 1] is a no-op on a gate target)
        p.penalty = {"structured_topn": L.PENALTY_STRUCTURED_TOPN, "mid": L.PENALTY_MID}.get(mode, L.PENALTY_NONE)
        p.penalty_coef = float(gate.mask_penalty_lr) * lam
    d = getattr(gate.cfg, "mask_binarize_decay", 0.0)
    p.binarize = float(d or 0.0)
    p.mask_lr = float(gate.cfg.mask_lr)
    p.apply_freeze = 0
    return p


def _all_reduce_mean(t: torch.Tensor) -> torch.Tensor:
    try:
        import torch.distributed as dist

        if dist.is_available() and dist.is_initialized():
            t = t.clone()
            dist.all_reduce(t, op=dist.ReduceOp.SUM)
            t.div_(dist.get_world_size())
    except Exception:
        pass
    return t


@torch.no_grad()
def glu_joint_update(gate_module, up_module, step, lambda_mid, sample_idx=None):
    """_update_glu_joint_mask(gate_module, up_module, step, lambda_mid) (:363-479).

    sample_idx optionally injects the tau sample (the reference draws it with
    torch.randint inside gate_module._tau_unstructured, :993).
    """
    if not gate_module.change_mask or gate_module.mask_type == "none":
        for m in (gate_module, up_module):
            m.weight.flipped_mask = 0
            m.weight.init_flipped_mask = 0
        return
    if step < int(gate_module.cfg.sparsity_warmup_steps):
        return
    K_ = max(1, int(gate_module._mask_update_period(step)))
    if step % K_ != 0:
        return
    if gate_module.mask.shape != up_module.mask.shape:
        warnings.warn(f"[GLU Joint] Shape mismatch: gate={gate_module.mask.shape}, up={up_module.mask.shape}. "
                      f"Falling back to independent update.")
        gate_module.update_mask(step, lambda_mid=lambda_mid)
        up_module.update_mask(step, lambda_mid=lambda_mid)
        return
    if gate_module.mask.numel() == 0:
        return
    ops_g, ops_u = gate_module._mask_operands(), up_module._mask_operands()
    code_g, code_u = gate_module._metric_code(ops_g), up_module._metric_code(ops_u)
    pg = gate_module._mask_params(step, ops_g, code_g) if gate_module.mask_type in ("unstructured", "structured") \
        else None
    pu = up_module._mask_params(step, ops_u, code_u) if up_module.mask_type in ("unstructured", "structured") \
        else None
    if pg is None or pu is None:  # only metric, eps and dtypes of these matter for the scores
        pg = pg or _score_only_params(gate_module, ops_g, code_g)
        pu = pu or _score_only_params(up_module, ops_u, code_u)
    s_dtype = torch.promote_types(*(torch.bfloat16 if p.score_dtype == L.DT_BF16 else torch.float32
                                    for p in (pg, pu)))
    S = K.joint_scores(pg, ops_g, pu, ops_u, s_dtype)

    rows, cols = S.shape
    mask_g, mask_u = gate_module.mask.detach(), up_module.mask.detach()
    frozen = ops_g.frozen
    p = _joint_params(gate_module, step, rows, cols, mask_g.dtype, frozen is not None, lambda_mid)
    ops_s = K.MaskOperands(weight=S, mask=S, hessian=S)
    stats = K.score_stats(p, ops_s)
    tau = None
    if p.gate == L.GATE_UNSTRUCTURED:
        if sample_idx is None:
            sample_idx = gate_module._sample_indices(S.numel(), S.device)
        tau = K.tau_quantile(p, ops_s, stats, gate_module._effective_sparsity(step), sample_idx)
        if not getattr(gate_module, "_in_summon_context", False):
            tau = _all_reduce_mean(tau)
    up_kind, up_n, _ = (L.HARD_THRESHOLD, 2, 4) if up_module._is_block_hard() else up_module._hard_kind()
    flips = torch.zeros(2, dtype=torch.int64, device=S.device)
    prev = [m.clone() if mod._is_block_hard() else None for m, mod in ((mask_g, gate_module), (mask_u, up_module))]
    K.glu_update_masks(p, S, mask_g, mask_u, frozen, stats, tau, up_kind, up_n,
                       None if prev[0] is not None else flips[0:1], None if prev[1] is not None else flips[1:2])
    for i, (m, mod) in enumerate(((mask_g, gate_module), (mask_u, up_module))):
        if prev[i] is not None:
            mod._flip_count(prev[i], m, flips[i:i + 1])

    hx = gate_module._hardening_schedule(step)
    gate_module.hardening_x = hx
    up_module.hardening_x = hx
    # the flip counts stay on the device until someone reads them (int() syncs)
    gate_module.weight.flipped_mask = flips[0]
    up_module.weight.flipped_mask = flips[1]
    for m in (gate_module, up_module):
        m.weight.init_flipped_mask = 0
        m.weight.mask = m.mask


def _score_only_params(module, ops, code) -> L.MaskParams:
    p = L.MaskParams()
    p.rows, p.cols = ops.weight.shape
    p.metric = code
    p.score_dtype = module._score_dtype(ops, code)
    p.eps_metric = 1e-8
    p.movement_temp = max(float(module.cfg.temperature), 1e-8)
    return p
