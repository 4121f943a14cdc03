"""One optimizer step of the sparse retraining loop on the drop-in ops.

Follows legacy/main_llama.py:1996-2211 for one process on one GPU (no
FSDP/DDP, no GradScaler: bf16 needs none):

  penalty = mid_penalty(student, lambda_mid)                     (:2047-2057)
          + sparsity_penalty(student, ratio, alpha)[0]           (:2059-2064)
      (the reference evaluates both in every micro-batch; they read only the
      frozen masks, so every micro-batch adds the same value)
  for each micro-batch (X, Y):                                   (:1996)
      logits, task, layerwise, kl = Distill_Model(X, Y)          (:2022)
      loss = h_task * task + h_kl * kl (+ h_sq * layerwise)       (:2025-2028)
      loss += penalty
      loss /= grad_accum                                         (:2067)
      all-finite check, else skip the step                       (:2074-2115)
      last micro-batch: update_hessian_hutchinson(student, loss) (:2111-2112)
      loss.backward()                                            (:2141)
  clip_grad_norm_(student.parameters(), grad_clip)               (:2170-2172)
  update_model_grad_ema(student, not hutchinson)                 (:2176-2177)
  optimizer lr <- schedule; optimizer.step(decay=...)            (:2180-2184)
  optimizer.zero_grad(set_to_none=True)                          (:2186)
  calculate_model_mask(student, iter_num, lambda_mid)            (:2211)

lambda_mid ramps to lambda_mid_max over 500 steps (2000 for the block
penalty modes), :2044-2052.  Each phase is bracketed by device events on the
current stream, so a caller can read a per-phase time breakdown without
extra synchronisation inside the step.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import utils as U
from .sparse_modeling import Distill_Model

PHASES = ("forward", "hutchinson", "backward", "optimizer", "mask_update")


@dataclass
class RetrainConfig:
    grad_accum: int = 1
    hardness_task: float = 1.0
    hardness_kldiv: float = 1.0
    hardness_squarehead: float = 0.0
    lambda_mid_max: float = 0.1
    sparsity_ratio: float = 0.5
    sparsity_alpha: float = 0.2
    grad_clip: float = 1.0
    hutchinson: bool = True
    mask_penalty_mode: str = "nm_2_4"
    autocast_dtype: torch.dtype | None = torch.bfloat16
    lr: float = 1e-4
    decay: float = 0.0


@dataclass
class StepResult:
    loss: float
    skipped: bool
    events: dict = field(default_factory=dict)

    def phase_ms(self) -> dict:
        """Milliseconds per phase (synchronises on the last event)."""
        ev = self.events
        if not ev:
            return {}
        ev["end"].synchronize()
        out = {}
        for name in PHASES:
            if name in ev:
                out[name] = sum(a.elapsed_time(b) for a, b in ev[name])
        return out


def lambda_mid_at(cfg: RetrainConfig, iter_num: int) -> float:
    warm = 2000 if cfg.mask_penalty_mode in ("block_sparse16", "block_sparse32", "block16") else 500
    if iter_num < warm:
        return cfg.lambda_mid_max * (iter_num / warm)
    return cfg.lambda_mid_max


class RetrainStep:
    """Callable step over (student, teacher, optimizer); `batches` is a list of grad_accum (X, Y) pairs."""

    def __init__(self, student, teacher, optimizer, cfg: RetrainConfig, timed: bool = False, on_grads=None):
        self.student = student
        self.model = Distill_Model(student, teacher)
        self.optimizer = optimizer
        self.cfg = cfg
        self.timed = timed
        self.on_grads = on_grads  # called with the student after clipping, before the optimizer step

    def _mark(self, events, name, start):
        if not self.timed:
            return None
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        if start is not None:
            events.setdefault(name, []).append((start, e))
        return e

    def __call__(self, iter_num: int, batches) -> StepResult:
        cfg = self.cfg
        if len(batches) != cfg.grad_accum:
            raise ValueError(f"expected {cfg.grad_accum} micro-batches, got {len(batches)}")
        ev: dict = {}
        lam = lambda_mid_at(cfg, iter_num)
        total = 0.0
        t = self._mark(ev, None, None)
        # The penalties read only the masks (frozen, no gradient), which change after the optimizer
        # step, not between micro-batches: each micro-batch's loss adds the same value, so it is
        # computed once per step (the reference recomputes it per micro-batch, :2047-2064).
        with U.shared_mask_rows():  # both read every mask's statistics: one pass over the masks
            penalty = U.mid_penalty(self.student, lam)
            if cfg.sparsity_alpha:
                pen, _cur = U.sparsity_penalty(self.student, target_sparsity=cfg.sparsity_ratio,
                                               alpha=cfg.sparsity_alpha)
                penalty = penalty + pen
        for micro, (X, Y) in enumerate(batches):
            last = micro == cfg.grad_accum - 1
            ctx = (torch.autocast("cuda", dtype=cfg.autocast_dtype) if cfg.autocast_dtype is not None
                   else torch.autocast("cuda", enabled=False))
            with ctx:
                _logits, task, layerwise, kl = self.model(X, Y)
                if task is None:
                    task = 0.0
                if layerwise is None:
                    loss = cfg.hardness_task * task + cfg.hardness_kldiv * kl
                else:
                    loss = cfg.hardness_task * task + cfg.hardness_squarehead * layerwise + cfg.hardness_kldiv * kl
                loss = loss + penalty
                loss = loss / cfg.grad_accum
            del _logits
            if not bool(torch.isfinite(loss.detach()).item()):
                self.optimizer.zero_grad(set_to_none=True)
                return StepResult(float("nan"), True)
            t = self._mark(ev, "forward", t)
            if cfg.hutchinson and last:
                U.update_hessian_hutchinson(self.student, loss)
                t = self._mark(ev, "hutchinson", t)
            loss.backward()
            total += float(loss.detach())
            t = self._mark(ev, "backward", t)
        if cfg.grad_clip:
            torch.nn.utils.clip_grad_norm_(self.student.parameters(), cfg.grad_clip)
        if self.on_grads is not None:
            self.on_grads(self.student)
        U.update_model_grad_ema(self.student, update_hessian_with_grad2=not cfg.hutchinson)
        for pg in self.optimizer.param_groups:
            pg["lr"] = cfg.lr
        self.optimizer.step(decay=cfg.decay)
        self.optimizer.zero_grad(set_to_none=True)
        t = self._mark(ev, "optimizer", t)
        U.calculate_model_mask(self.student, iter_num, lambda_mid=lam)
        t = self._mark(ev, "mask_update", t)
        if self.timed:
            ev["end"] = t
        return StepResult(total, False, ev)


def optimizer_groups(model, weight_decay: float):
    """Parameter groups of the reference's configure_optimizers (legacy/model_llama.py:150-158):
    >= 2-D parameters decay, the rest do not."""
    params = [p for p in model.parameters() if p.requires_grad]
    return [{"params": [p for p in params if p.dim() >= 2], "weight_decay": weight_decay},
            {"params": [p for p in params if p.dim() < 2], "weight_decay": 0.0}]
