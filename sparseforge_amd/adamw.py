"""Drop-in AdamW with the mask-aware decay: one fused pass over all parameters of a step.

Mirrors legacy/adamw.py of liuhanzuo/SparseForge: the same constructor
(``AdamW(params, lr, betas, eps, weight_decay, amsgrad, srste_decay,
adaptive_l1_decay)``), the same ValueErrors, the same ``step(closure=None,
decay=None)`` (``decay`` stays a keyword so ``scaler.step(optimizer,
decay=...)`` works), and the same per-parameter state names (``step``,
``exp_avg``, ``exp_avg_sq``, ``max_exp_avg_sq``), so checkpoints move between
the two.  The masked decay finds the mask through the parameter's ``mask``
attribute, which SparseLinear aliases to its mask (sparse_modeling.py:372).

Each parameter's whole update (decoupled weight decay, masked decay,
moments, bias corrections, AMSGrad, adaptive L1) is one elementwise pass;
``step`` updates all parameters that share dtypes and hyper-parameters with
one ``sf_adamw_step_multi`` call (a launch per 40 tensors, the tensor table
in the kernel arguments).  Parameters must live on the GPU (there is no CPU
path).
"""
from __future__ import annotations

import torch

from . import _lib as L
from . import profiling as _prof


def _code(t: torch.Tensor) -> int:
    return L.dtype_code(t)


def adamw_step_(p: torch.Tensor, grad: torch.Tensor, exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor,
                max_exp_avg_sq: torch.Tensor | None, mask: torch.Tensor | None, step: int, lr: float, betas, eps: float,
                weight_decay: float, decay: float = 0.0, l1: float = 0.0, amsgrad: bool = False,
                apply_l1: bool | None = None, bf16_copy: torch.Tensor | None = None) -> None:
    """In-place fused AdamW step of one tensor (``step`` = count after this step)."""
    dev = L.require_device(p, grad, exp_avg, exp_avg_sq, max_exp_avg_sq, mask, bf16_copy)
    n = p.numel()
    for name, t in (("grad", grad), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq), ("max_exp_avg_sq", max_exp_avg_sq),
                    ("mask", mask), ("bf16_copy", bf16_copy)):
        if t is not None and t.numel() != n:
            raise ValueError(f"adamw: {name} has {t.numel()} elements, the parameter {n}")
    if exp_avg.dtype != exp_avg_sq.dtype or (max_exp_avg_sq is not None and max_exp_avg_sq.dtype != exp_avg.dtype):
        raise TypeError("adamw: optimizer state tensors must share one dtype")
    if bf16_copy is not None and bf16_copy.dtype != torch.bfloat16:
        raise TypeError("adamw: the parameter copy must be bfloat16")
    hp = L.AdamwParams()
    hp.lr, hp.weight_decay, hp.beta1, hp.beta2, hp.eps = float(lr), float(weight_decay), float(betas[0]), \
        float(betas[1]), float(eps)
    hp.decay, hp.l1, hp.amsgrad, hp.step = float(decay), float(l1), int(bool(amsgrad)), int(step)
    hp.apply_l1 = int(p.dim() >= 2 if apply_l1 is None else bool(apply_l1))
    nbytes = n * (2 * p.element_size() + grad.element_size() + 4 * exp_avg.element_size()
                  + (2 * exp_avg.element_size() if amsgrad else 0) + (mask.element_size() if mask is not None else 0)
                  + (2 if bf16_copy is not None else 0))
    with _prof.region("sf_adamw_step", nbytes, "B", dev):
        L.check(L.lib().sf_adamw_step(L.ptr(p), _code(p), L.ptr(grad), _code(grad), L.ptr(exp_avg), L.ptr(exp_avg_sq),
                                      L.ptr(max_exp_avg_sq), _code(exp_avg), L.ptr(mask),
                                      _code(mask) if mask is not None else L.DT_F32, L.ptr(bf16_copy), n,
                                      L.byref(hp), L.stream(dev)), "sf_adamw_step")


class TensorStep:
    """Operands of one tensor in a multi-tensor step (see adamw_step_multi_)."""

    __slots__ = ("param", "grad", "exp_avg", "exp_avg_sq", "max_exp_avg_sq", "mask", "bf16_copy", "apply_l1")

    def __init__(self, param, grad, exp_avg, exp_avg_sq, max_exp_avg_sq=None, mask=None, bf16_copy=None,
                 apply_l1=None):
        self.param, self.grad, self.exp_avg, self.exp_avg_sq = param, grad, exp_avg, exp_avg_sq
        self.max_exp_avg_sq, self.mask, self.bf16_copy = max_exp_avg_sq, mask, bf16_copy
        self.apply_l1 = param.dim() >= 2 if apply_l1 is None else bool(apply_l1)


def adamw_step_multi_(items, step: int, lr: float, betas, eps: float, weight_decay: float, decay: float = 0.0,
                      l1: float = 0.0, amsgrad: bool = False) -> None:
    """In-place fused AdamW step of every TensorStep in `items` (one parameter dtype, one state dtype,
    one step count): one sf_adamw_step_multi call, one launch per 40 tensors."""
    items = [t for t in items if t.param.numel() > 0]
    if not items:
        return
    dev = L.require_device(items[0].param)
    pdt, sdt = items[0].param.dtype, items[0].exp_avg.dtype
    arr = (L.AdamwTensor * len(items))()
    nbytes = 0
    for e, t in zip(arr, items):
        L.require_device(t.param, t.grad, t.exp_avg, t.exp_avg_sq, t.max_exp_avg_sq, t.mask, t.bf16_copy)
        n = t.param.numel()
        if t.param.device != dev or t.param.dtype != pdt or t.exp_avg.dtype != sdt or t.exp_avg_sq.dtype != sdt:
            raise TypeError("adamw: a multi-tensor step needs one device, one parameter dtype and one state dtype")
        for name, x in (("grad", t.grad), ("exp_avg", t.exp_avg), ("exp_avg_sq", t.exp_avg_sq),
                        ("max_exp_avg_sq", t.max_exp_avg_sq), ("mask", t.mask), ("bf16_copy", t.bf16_copy)):
            if x is not None and x.numel() != n:
                raise ValueError(f"adamw: {name} has {x.numel()} elements, the parameter {n}")
        if amsgrad and (t.max_exp_avg_sq is None or t.max_exp_avg_sq.dtype != sdt):
            raise TypeError("adamw: amsgrad needs max_exp_avg_sq in the state dtype")
        if t.bf16_copy is not None and t.bf16_copy.dtype != torch.bfloat16:
            raise TypeError("adamw: the parameter copy must be bfloat16")
        e.param, e.grad, e.exp_avg, e.exp_avg_sq = L.ptr(t.param), L.ptr(t.grad), L.ptr(t.exp_avg), L.ptr(t.exp_avg_sq)
        e.max_exp_avg_sq = L.ptr(t.max_exp_avg_sq) if amsgrad else None
        e.mask, e.param_bf16_copy, e.n = L.ptr(t.mask), L.ptr(t.bf16_copy), n
        e.grad_dtype = _code(t.grad)
        e.mask_dtype = _code(t.mask) if t.mask is not None else L.DT_F32
        e.apply_l1 = int(t.apply_l1)
        nbytes += n * (2 * t.param.element_size() + t.grad.element_size() + 4 * t.exp_avg.element_size()
                       + (2 * t.exp_avg.element_size() if amsgrad else 0)
                       + (t.mask.element_size() if t.mask is not None else 0) + (2 if t.bf16_copy is not None else 0))
    hp = L.AdamwParams()
    hp.lr, hp.weight_decay, hp.beta1, hp.beta2, hp.eps = float(lr), float(weight_decay), float(betas[0]), \
        float(betas[1]), float(eps)
    hp.decay, hp.l1, hp.amsgrad, hp.step, hp.apply_l1 = float(decay), float(l1), int(bool(amsgrad)), int(step), 0
    with _prof.region("sf_adamw_step_multi", nbytes, "B", dev):
        L.check(L.lib().sf_adamw_step_multi(arr, len(items), L.dtype_code(items[0].param), L.dtype_code(items[0].exp_avg),
                                            L.byref(hp), L.stream(dev)), "sf_adamw_step_multi")


class AdamW(torch.optim.Optimizer):
    """AdamW with SR-STE masked decay and adaptive L1 decay (legacy/adamw.py:13-176)."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2, amsgrad=False,
                 srste_decay=None, adaptive_l1_decay=0.0):
        if not 0.0 <= lr:
            raise ValueError("Invalid learning rate: {}".format(lr))
        if not 0.0 <= eps:
            raise ValueError("Invalid epsilon value: {}".format(eps))
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError("Invalid beta parameter at index 0: {}".format(betas[0]))
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError("Invalid beta parameter at index 1: {}".format(betas[1]))
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, amsgrad=amsgrad)
        self.decay = srste_decay if srste_decay is not None else 0.0
        self.adaptive_l1_decay = float(adaptive_l1_decay) if adaptive_l1_decay is not None else 0.0
        super().__init__(params, defaults)

    def __setstate__(self, state):
        super().__setstate__(state)
        for group in self.param_groups:
            group.setdefault("amsgrad", False)

    @torch.no_grad()
    def step(self, closure=None, decay=None):
        """One step of every parameter with a gradient (:65-176).

        Parameters that share a device, dtypes, hyper-parameters and step count
        are updated by one sf_adamw_step_multi call (one pass over HBM for the
        whole group) instead of one kernel per parameter."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        if decay is not None:
            self.decay = decay
        groups: dict = {}
        keep = []  # temporaries (contiguous gradient copies, mask views) alive until their launch
        for group in self.param_groups:
            lr, betas, eps, wd, amsgrad = group["lr"], group["betas"], group["eps"], group["weight_decay"], \
                group["amsgrad"]
            for p in group["params"]:
                if p.grad is None:
                    continue
                grad = p.grad
                if grad.shape != p.shape:
                    # sharded / flattened views: align when the element counts agree (:90-96)
                    if grad.numel() == p.numel() and p.numel() > 0:
                        grad = grad.view_as(p)
                    else:
                        p.mul_(1 - lr * wd)  # the reference applies the decoupled decay, then skips
                        continue
                mask = getattr(p, "mask", None)
                if mask is not None and mask.shape != p.shape:
                    mask = mask.view_as(p) if (mask.numel() == p.numel() and p.numel() > 0) else None
                state = self.state[p]
                if len(state) == 0:
                    state["step"] = 0
                    state["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    if amsgrad:
                        state["max_exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                if state["exp_avg"].shape != p.shape:  # resumed across a different sharding (:134-141)
                    state["exp_avg"] = torch.zeros_like(p)
                    state["exp_avg_sq"] = torch.zeros_like(p)
                    state["step"] = 0
                    if amsgrad and "max_exp_avg_sq" in state:
                        state["max_exp_avg_sq"] = torch.zeros_like(p)
                if amsgrad and "max_exp_avg_sq" not in state:
                    state["max_exp_avg_sq"] = torch.zeros_like(p)
                state["step"] += 1
                g = grad.contiguous()
                m = mask.detach().contiguous() if mask is not None else None
                keep.extend(t for t in (g, m) if t is not None)
                key = (p.device, p.dtype, state["exp_avg"].dtype, state["step"], float(lr), tuple(map(float, betas)),
                       float(eps), float(wd), bool(amsgrad))
                groups.setdefault(key, []).append(
                    TensorStep(p.data, g, state["exp_avg"], state["exp_avg_sq"],
                               state.get("max_exp_avg_sq") if amsgrad else None, m, apply_l1=p.dim() >= 2))
        for (_dev, _pdt, _sdt, step, lr, betas, eps, wd, amsgrad), items in groups.items():
            adamw_step_multi_(items, step, lr, betas, eps, wd, decay=float(self.decay),
                              l1=float(self.adaptive_l1_decay), amsgrad=amsgrad)
        del keep
        return loss
