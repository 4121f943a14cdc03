"""Drop-in model-level mask operations (legacy/utils.py of liuhanzuo/SparseForge).

Same function names, signatures and side effects as the reference's
hot-path helpers:

  get_raw_model, set_model_mode, sync_weight, initialize_model      (:58-116)
  update_model_grad_ema                                            (:123-134)
  calculate_model_mask (with the GLU gate/up joint update)         (:184-643)
  calculate_flip_rate                                              (:692-704)
  _rademacher_like, update_hessian_hutchinson                      (:710-869)
  _compute_importance_scores, _compute_joint_gate_target           (:482-613)
  update_mask_penalty_lr                                           (:142-180)
  mid_penalty, sparsity_penalty, nm_2_4_tile_stats, harden_fraction (:876-1276)
  mask_stats, log_mask_stats                                       (:2069-2335)

The tensor work runs in the sparseforge_amd HIP library; FSDP handling of
the reference (summon_full_params, sharded views) does not apply to the
single-GPU path and is left out.
"""
from __future__ import annotations

import contextlib
import itertools
import re

import torch

from . import _lib as L
from . import kernels as K
from . import profiling as _prof
from .sparse_modeling import SparseLinear, draw_samples

_nullctx = contextlib.nullcontext

_seed_counter = itertools.count(1)


@torch.no_grad()
def get_raw_model(model):
    """Unwrap DDP (.module) and Distill_Model (.student) wrappers (:58-88)."""
    if hasattr(model, "_fsdp_wrapped_module"):
        inner = model._fsdp_wrapped_module
        if hasattr(inner, "student"):
            st = inner.student
            return st._fsdp_wrapped_module if hasattr(st, "_fsdp_wrapped_module") else st
        return inner
    if hasattr(model, "module"):
        return model.module.student if hasattr(model.module, "student") else model.module
    if hasattr(model, "student"):
        st = model.student
        return st._fsdp_wrapped_module if hasattr(st, "_fsdp_wrapped_module") else st
    return model


def _sparse_modules(model):
    raw = get_raw_model(model)
    return [(n, m) for n, m in raw.named_modules() if isinstance(m, SparseLinear)]


@torch.no_grad()
def set_model_mode(model, mode: str):
    for _, m in _sparse_modules(model):
        m.mode = mode


@torch.no_grad()
def sync_weight(model, device=None):
    if device is not None:
        model = model.to(device)
    for _, m in _sparse_modules(model):
        m.sync_weight()


@torch.no_grad()
def initialize_model(model):
    for _, m in _sparse_modules(model):
        m.initialize()
        if getattr(m, "SLoRB", False):
            m.init_SLoRB()


def update_mask_penalty_lr(model, step: int, max_steps: int, penalty_lr_min: float, penalty_lr_max: float,
                           schedule: str = "linear"):
    """Set every SparseLinear's mask_penalty_lr from a constant / linear / cosine ramp from
    penalty_lr_min (step 0) to penalty_lr_max (max_steps) and return it (:142-180)."""
    import math

    progress = min(1.0, step / max(1, max_steps))
    if schedule == "linear":
        lr = penalty_lr_min + (penalty_lr_max - penalty_lr_min) * progress
    elif schedule == "cosine":
        lr = penalty_lr_min + (penalty_lr_max - penalty_lr_min) * (0.5 * (1.0 - math.cos(math.pi * progress)))
    else:  # 'constant' and anything unknown
        lr = penalty_lr_max
    for _, m in _sparse_modules(model):
        m.mask_penalty_lr = lr
    return lr


@torch.no_grad()
def update_model_grad_ema(model, update_hessian_with_grad2: bool = True):
    for _, m in _sparse_modules(model):
        m.update_grad_hessian_ema(update_hessian_with_grad2=update_hessian_with_grad2)


def _identify_glu_pairs(sparse_modules_dict):
    """{gate_name: up_name} for `*.mlp.gate_proj`/`up_proj` and `*.mlp.w1`/`w3` pairs (:313-361)."""
    pairs = {}
    for gate_re, up_leaf in ((r"(.+\.mlp)\.gate_proj$", "up_proj"), (r"(.+\.mlp)\.w1$", "w3")):
        pat = re.compile(gate_re)
        for name, mod in sparse_modules_dict.items():
            mt = pat.match(name)
            if not mt:
                continue
            up = f"{mt.group(1)}.{up_leaf}"
            if up in sparse_modules_dict and getattr(mod.cfg, "glu_joint_mask", False):
                pairs[name] = up
    return pairs


def calculate_model_mask(model, step=0, lambda_mid: float = 0.0):
    """Periodic mask update of every SparseLinear (:184-310); gate/up pairs share one target when
    glu_joint_mask is set."""
    mods = dict(_sparse_modules(model))
    any_update = False
    for m in mods.values():
        if (not m.change_mask) or m.mask_type == "none":
            continue
        if step < int(m.cfg.sparsity_warmup_steps):
            continue
        if step % max(1, int(m._mask_update_period(step))) != 0:
            continue
        any_update = True
        break
    if not any_update:
        return
    pairs = _identify_glu_pairs(mods) if any(getattr(m.cfg, "glu_joint_mask", False) for m in mods.values()) else {}
    handled = set(pairs) | set(pairs.values())
    for m in mods.values():
        m._in_summon_context = False
    # GLU pairs and the staged block-type updates run on a few side streams and overlap
    devs = {m.mask.device for m in mods.values()}
    pipe = K.LayerPipeline(next(iter(devs))) if len(devs) == 1 and next(iter(devs)).type == "cuda" else None
    for gate_name, up_name in pairs.items():
        with pipe.next() if pipe else _nullctx():
            _update_glu_joint_mask(mods[gate_name], mods[up_name], step, lambda_mid)
    # Layers on the fused update path whose parameters differ only in shape update together
    # (sf_update_mask_multi: a few launches per 28 layers, results equal to one update_mask per
    # layer); the block hard types and block penalty modes keep their multi-pass update.
    batches: dict = {}
    draws: dict = {}    # (device, sample size) -> [(size, numel, seed)] of the batched layers
    samples: dict = {}  # id of a draw -> its sorted sample
    for name, m in mods.items():
        if name in handled:
            continue
        prep = m._prepare_update(step, lambda_mid)
        if prep is None:
            continue
        ops, p, code = prep
        if m._staged_update(p):
            with pipe.next() if pipe else _nullctx():
                stats, tau = m._gate_inputs(step, ops, code, p)
                flips = torch.zeros(1, dtype=torch.int64, device=m.mask.device)
                m._update_mask_staged(step, ops, p, stats, tau, flips)
                m._finish_update(step, flips)
            continue
        q = float(m._effective_sparsity(step)) if p.gate == L.GATE_UNSTRUCTURED else 0.0
        shape_free = L.MaskParams.from_buffer_copy(p)
        shape_free.rows = shape_free.cols = 0
        key = (ops.device(), tuple(ops.dt(t) if t is not None else -1
                                   for t in (ops.weight, ops.hessian, ops.aux, ops.mask, ops.frozen)),
               bytes(shape_free), q)
        # the tau sample's seed, drawn here so every layer (staged or batched) draws in module order, as one
        # update_mask per layer does; the samples themselves are generated below, several lists per launch
        seed = m._sample_seed(ops.weight.numel()) if p.gate == L.GATE_UNSTRUCTURED else None
        idx = None
        if seed is not None:
            idx = (m._sample_size(ops.weight.numel()), ops.weight.numel(), seed)
            draws.setdefault((ops.device(), idx[0]), []).append(idx)
        batches.setdefault(key, []).append([m, ops, p, idx])
    for (dev, size), lists in draws.items():
        rows = draw_samples(size, [n for _, n, _ in lists], [s for _, _, s in lists], dev)
        for r, spec in enumerate(lists):
            samples[id(spec)] = rows[r]
    for (dev, _dts, _pb, q), items in batches.items():
        for it in items:
            it[3] = samples[id(it[3])] if it[3] is not None else None
        n = len(items)
        stats = torch.empty((n, 2), dtype=torch.float32, device=dev)
        tau = torch.empty(n, dtype=torch.float32, device=dev)
        flips = torch.zeros(n, dtype=torch.int64, device=dev)
        jobs = [K.MaskJob(ops, idx, stats[i], tau[i:i + 1], flips[i:i + 1])
                for i, (m, ops, p, idx) in enumerate(items)]
        K.update_mask_multi(items[0][2], q, jobs)
        for i, (m, _ops, _p, _idx) in enumerate(items):
            m._finish_update(step, flips[i:i + 1])
    if pipe:
        pipe.join()


@torch.no_grad()
def _update_glu_joint_mask(gate_module, up_module, step, lambda_mid, sample_idx=None):
    """Joint gate/up mask update (:363-479): one target G from the summed scores, EMA'd into both masks."""
    from .glu import glu_joint_update

    glu_joint_update(gate_module, up_module, step, lambda_mid, sample_idx)


@torch.no_grad()
def _compute_importance_scores(module):
    """A SparseLinear's importance scores (:482-533), in the dtype the reference's torch ops produce
    (the promotion of W and the metric's operand), on the device (sf_importance_scores)."""
    from .glu import _score_only_params

    ops = module._mask_operands()
    code = module._metric_code(ops)  # hessian_obd without H: W * W, as :506-511
    p = _score_only_params(module, ops, code)
    dt = torch.bfloat16 if p.score_dtype == L.DT_BF16 else torch.float32
    return K.importance_scores(p, ops, dt)


@torch.no_grad()
def _compute_joint_gate_target(module, scores, step, sample_idx=None):
    """Gate target G of `module` from precomputed (joint) scores (:536-613): z-scores in the mask
    dtype, the module's gate form at the step's temperature (unstructured tau over a sample of z,
    structured top-N), the beta structural mix and the frozen override.  `sample_idx` optionally
    injects the tau sample (the reference draws it with torch.randint, :993)."""
    from .glu import _joint_params

    if scores.numel() == 0:
        return module.mask
    S = scores.detach().contiguous()
    if S.shape != module.mask.shape:
        raise ValueError(f"scores shape {tuple(S.shape)} != mask shape {tuple(module.mask.shape)}")
    mask = module.mask.data
    frozen = module._mask_operands().frozen
    rows, cols = S.shape
    p = _joint_params(module, step, rows, cols, mask.dtype, frozen is not None, 0.0)
    ops = K.MaskOperands(weight=S, mask=mask, hessian=S, frozen=frozen)
    stats = K.score_stats(p, ops)
    tau = None
    if p.gate == L.GATE_UNSTRUCTURED:
        if sample_idx is None:
            sample_idx = module._sample_indices(S.numel(), S.device)
        tau = K.tau_quantile(p, ops, stats, module._effective_sparsity(step), sample_idx)
    return K.gate_target(p, ops, stats, tau, mask.dtype)


@torch.no_grad()
def calculate_flip_rate(model):
    """(flipped, ratio, init_flipped, init_ratio) summed over SparseLinear layers (:692-704)."""
    flipped = init_flipped = total = 0
    for _, m in _sparse_modules(model):
        flipped += int(getattr(m.weight, "flipped_mask", 0))
        init_flipped += int(getattr(m.weight, "init_flipped_mask", 0))
        total += int(getattr(m.weight, "param_count", m.weight.numel()))
    return flipped, flipped / max(total, 1), init_flipped, init_flipped / max(total, 1)


# ---------------------------------------------------------------------------
# Hutchinson Hessian diagonal (:710-869)
# ---------------------------------------------------------------------------
def rademacher(shape, dtype, device, seed: int) -> torch.Tensor:
    """+-1 probe from the counter-based generator: v_i = f(seed, i) (sf_rademacher)."""
    v = torch.empty(shape, dtype=dtype, device=device)
    L.check(L.lib().sf_rademacher(L.ptr(v), L.dtype_code(v), v.numel(), seed & ((1 << 64) - 1), L.stream(device)),
            "sf_rademacher")
    return v


def _rademacher_like(t: torch.Tensor, seed: int | None = None) -> torch.Tensor:
    """+-1 tensor like t (the reference draws torch.randint, :710-711; here the counter RNG)."""
    return rademacher(t.shape, t.dtype, t.device, next(_seed_counter) if seed is None else seed)


class _ProbeDot(torch.autograd.Function):
    """sum(g * v(seed)) with v regenerated on the fly; backward gives grad_out * v."""

    @staticmethod
    def forward(ctx, g, seed, v):
        dev = L.require_device(g)
        g = g.contiguous()
        ws = torch.empty(L.lib().sf_rademacher_dot_workspace_size(), dtype=torch.uint8, device=dev)
        out = torch.empty((), dtype=torch.float32, device=dev)
        L.check(L.lib().sf_rademacher_dot(L.ptr(g), L.dtype_code(g), L.ptr(v), L.dtype_code(v) if v is not None else 0,
                                          g.numel(), seed, L.ptr(out), L.ptr(ws), ws.numel(), L.stream(dev)),
                "sf_rademacher_dot")
        ctx.seed, ctx.shape, ctx.dtype = seed, g.shape, g.dtype
        ctx.save_for_backward(v)
        return out.to(g.dtype)

    @staticmethod
    def backward(ctx, grad_out):
        (v,) = ctx.saved_tensors
        if v is None:
            v = rademacher(ctx.shape, ctx.dtype, grad_out.device, ctx.seed)
        return grad_out * v, None, None


def hutchinson_update_(H: torch.Tensor, hvp: torch.Tensor, beta: float, seed: int = 0,
                       v: torch.Tensor | None = None) -> None:
    """H <- beta H + (1 - beta) clamp(hvp * v, 0) in one pass (v from seed, or explicit)."""
    dev = L.require_device(H, hvp, v)
    if hvp.numel() != H.numel() or (v is not None and v.numel() != H.numel()):
        raise ValueError("hutchinson: hvp / v / hessian_diag sizes differ")
    nbytes = H.numel() * (2 * H.element_size() + hvp.element_size() + (v.element_size() if v is not None else 0))
    with _prof.region("sf_hutchinson_update", nbytes, "B", dev):
        L.check(L.lib().sf_hutchinson_update(L.ptr(H), L.dtype_code(H), L.ptr(hvp.contiguous()), L.dtype_code(hvp),
                                             L.ptr(v), L.dtype_code(v) if v is not None else 0, H.numel(),
                                             seed & ((1 << 64) - 1), float(beta), L.stream(dev)),
                "sf_hutchinson_update")


def hutchinson_update_multi_(items) -> None:
    """hutchinson_update_ over many (H, hvp, beta, seed) with regenerated probes in a few launches
    (sf_hutchinson_update_multi: 48 tensors per launch); every element gets the single call's value.
    Items whose sizes are not multiples of 4 take the single call."""
    groups: dict = {}
    for H, hvp, beta, seed in items:
        hvp = hvp.contiguous()
        L.require_device(H, hvp)
        if hvp.numel() != H.numel():
            raise ValueError("hutchinson: hvp / hessian_diag sizes differ")
        if H.numel() % 4 or H.data_ptr() % 16 or hvp.data_ptr() % 16:
            hutchinson_update_(H, hvp, beta, seed=seed)
            continue
        groups.setdefault((H.device, H.dtype, hvp.dtype), []).append((H, hvp, beta, seed))
    for (dev, hdt, gdt), grp in groups.items():
        table = (L.HutchTensor * len(grp))()
        nbytes = 0
        for i, (H, hvp, beta, seed) in enumerate(grp):
            e = table[i]
            e.H, e.hvp, e.n = L.ptr(H), L.ptr(hvp), H.numel()
            e.seed, e.beta = seed & ((1 << 64) - 1), float(beta)
            nbytes += H.numel() * (2 * H.element_size() + hvp.element_size())
        with _prof.region("sf_hutchinson_update_multi", nbytes, "B", dev):
            L.check(L.lib().sf_hutchinson_update_multi(table, len(grp), L.dtype_code(grp[0][0]),
                                                       L.dtype_code(grp[0][1]), L.stream(dev)),
                    "sf_hutchinson_update_multi")


def update_hessian_hutchinson(model, loss, probes=None):
    """Hutchinson update of every SparseLinear's hessian_diag (:714-869); call before loss.backward().

    probes: optional list of explicit +-1 tensors, one per SparseLinear weight in
    module order (parity tests feed the reference's own draws); by default each
    weight's probe comes from the counter RNG with a fresh seed.
    """
    owners = [m for _, m in _sparse_modules(model)]
    if not owners:
        return
    params = [m.weight for m in owners]
    try:
        grads = torch.autograd.grad(loss, params, create_graph=True, retain_graph=True, allow_unused=True)
        seeds, vs, dot = [], [], None
        for k, (g, p) in enumerate(zip(grads, params)):
            if g is None:
                seeds.append(None)
                vs.append(None)
                continue
            seed = next(_seed_counter)
            v = probes[k].to(device=p.device, dtype=p.dtype).contiguous() if probes is not None else None
            seeds.append(seed)
            vs.append(v)
            term = _ProbeDot.apply(g, seed, v)
            dot = term if dot is None else dot + term
        hvps = [None] * len(params) if dot is None else torch.autograd.grad(dot, params, retain_graph=True,
                                                                             allow_unused=True)
    except RuntimeError as e:
        raise RuntimeError(
            f"[Hutchinson] Double-backward failed: {e}\n"
            f"This usually means Flash Attention (SDPA) is enabled. "
            f"Set --eager_attention True to use Hutchinson Hessian estimation."
        ) from e
    try:
        import torch.distributed as dist

        world = dist.get_world_size() if dist.is_available() and dist.is_initialized() else 1
    except Exception:
        world = 1
    with torch.no_grad():
        batched = []  # probes regenerated from their seeds: one multi-tensor update
        for m, hvp, seed, v in zip(owners, hvps, seeds, vs):
            if hvp is None or seed is None or m._is_placeholder("hessian_diag"):
                continue
            beta = float(getattr(m.cfg, "beta", 0.99))
            if world == 1 and v is None:
                batched.append((m.hessian_diag.data, hvp.detach(), beta, seed))
                continue
            if world > 1:
                # data-parallel ranks average their estimates before the EMA (:863-865)
                vv = v if v is not None else rademacher(hvp.shape, hvp.dtype, hvp.device, seed)
                est = (hvp * vv).clamp_(min=0.0)
                dist.all_reduce(est, op=dist.ReduceOp.SUM)
                est.div_(world)
                hutchinson_update_(m.hessian_diag.data, est, beta, v=torch.ones_like(est))
            else:
                hutchinson_update_(m.hessian_diag.data, hvp.detach(), beta, seed=seed, v=v)
        if batched:
            hutchinson_update_multi_(batched)


# ---------------------------------------------------------------------------
# Penalties and mask statistics (:876-1234, :2069-2335).  Every mask is read
# once by sf_mask_stats (all sums of a layer in one fused pass, kept on the
# device); the scalars are composed from the per-layer rows exactly as the
# reference composes its per-layer torch reductions, with one host read at
# the point where the reference itself calls .item().
# ---------------------------------------------------------------------------
def _model_device(model):
    for p in get_raw_model(model).parameters():
        return p.device
    return torch.device("cpu")


def _dist_sum(*tensors):
    """All-reduce (sum) over the data-parallel group when one is initialised."""
    try:
        import torch.distributed as dist

        if dist.is_available() and dist.is_initialized():
            for t in tensors:
                dist.all_reduce(t, op=dist.ReduceOp.SUM)
    except Exception:
        pass


_ROWS_MEMO: dict | None = None


@contextlib.contextmanager
def shared_mask_rows():
    """Within the block, statistics rows of a mask list are computed once: a second request for the same
    masks (same storage, version, shape, dtype and tail) gets the first one's rows.  The retraining step
    wraps mid_penalty and sparsity_penalty in it (both read every mask of the model, unchanged between
    them)."""
    global _ROWS_MEMO
    prev, _ROWS_MEMO = _ROWS_MEMO, {}
    try:
        yield
    finally:
        _ROWS_MEMO = prev


def _mask_rows(masks, tails=None, eps: float = 1e-8):
    """[len(masks), MSTAT_COUNT] float64 on the masks' device: sf_mask_stats of each mask."""
    key = None
    if _ROWS_MEMO is not None:
        key = (eps,) + tuple((m.data_ptr(), m._version, tuple(m.shape), m.dtype, 0 if tails is None else int(tails[i]))
                             for i, m in enumerate(masks))
        if key in _ROWS_MEMO:
            return _ROWS_MEMO[key]
    dev = masks[0].device
    rows = torch.empty((len(masks), L.MSTAT_COUNT), dtype=torch.float64, device=dev)
    ws = K.mask_stats_workspace(dev)
    for i, m in enumerate(masks):
        K.mask_stats(m.contiguous(), rows[i], 0 if tails is None else int(tails[i]), eps, ws)
    if key is not None:
        _ROWS_MEMO[key] = rows
    return rows


def _round_sum_to(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """f64 sums as torch's .sum() of a tensor of `dtype` returns them (f32 accumulation, result in dtype)."""
    return x.to(torch.float32).to(dtype).to(torch.float64)


@torch.no_grad()
def mid_penalty(model, lambda_mid: float = 0.0):
    """lambda_mid * mean(mask * (1 - mask)) over all SparseLinear masks (:876-938); layers whose mask
    holds NaN or inf are left out; 0-dim float32 tensor on the model's device."""
    device = _model_device(model)
    if lambda_mid <= 0:
        return torch.tensor(0.0, device=device)
    masks = [m.mask.detach() for _, m in _sparse_modules(model) if m.mask.numel() > 0]
    total_penalty = torch.zeros((), device=device, dtype=torch.float64)
    total_count = torch.zeros((), device=device, dtype=torch.float64)
    if masks:
        rows = _mask_rows(masks)
        ok = rows[:, L.MSTAT_NONFINITE] == 0
        local = torch.stack([_round_sum_to(rows[i, L.MSTAT_MID], m.dtype) for i, m in enumerate(masks)])
        numel = torch.tensor([float(m.numel()) for m in masks], dtype=torch.float64, device=rows.device)
        total_penalty += torch.where(ok, local, torch.zeros_like(local)).sum().to(device)
        total_count += torch.where(ok, numel, torch.zeros_like(numel)).sum().to(device)
    _dist_sum(total_penalty, total_count)
    count_v = float(total_count.item())
    if count_v <= 0:
        return torch.tensor(0.0, device=device)
    result = lambda_mid * (total_penalty / count_v)
    if torch.isnan(result) or torch.isinf(result):
        return torch.tensor(0.0, device=device)
    return result.to(dtype=torch.float32)


@torch.no_grad()
def sparsity_penalty(model, target_sparsity: float = 0.5, alpha: float = 0.0):
    """(alpha * (sparsity - target)^2 as a tensor, sparsity) (:942-1025).  structured masks count
    M - N pruned per full group of M plus the threshold tail; the rest count mask < 0.5."""
    device = _model_device(model)
    cnt = torch.zeros((), device=device, dtype=torch.float64)
    tot = torch.zeros((), device=device, dtype=torch.float64)
    masks, tails, slots, const_cnt, const_tot = [], [], [], 0.0, 0.0
    for _, module in _sparse_modules(model):
        m = module.mask.detach()
        if m.numel() == 0:
            continue
        if getattr(module, "mask_type", "unstructured") == "structured" and m.dim() == 2:
            N, M = int(getattr(module, "N", 2)), int(getattr(module, "M", 4))
            out_dim, in_dim = m.shape
            in_full = (in_dim // M) * M
            if in_full > 0:
                const_tot += float(out_dim * in_full)
                const_cnt += float(out_dim * (in_full // M) * (M - N))
                if in_full < in_dim:
                    const_tot += float(out_dim * (in_dim - in_full))
                    masks.append(m), tails.append(in_full), slots.append(L.MSTAT_TAIL_LT05)
                continue
        const_tot += float(m.numel())
        masks.append(m), tails.append(0), slots.append(L.MSTAT_LT05)
    cnt += const_cnt
    tot += const_tot
    if masks:
        rows = _mask_rows(masks, tails)
        sel = torch.tensor(slots, device=rows.device)
        cnt += rows.gather(1, sel[:, None]).sum().to(device)
    _dist_sum(cnt, tot)
    tot_v = float(tot.item())
    cur = 0.0 if tot_v <= 0 else float((cnt / tot).item())
    pen = torch.tensor(0.0, device=device)
    if alpha != 0.0:
        diff = cur - float(target_sparsity)
        pen = torch.tensor(float(alpha * (diff * diff)), device=device)
    return pen, cur


def _tile_view(module, m):
    """(rows, cols) over which nm_2_4_tile_stats groups a mask by 4 along the last dim, or None (:1089-1146)."""
    M = 4
    if m.dim() == 2:
        return (m.shape[0], m.shape[1]) if m.shape[1] >= M else None
    if m.dim() == 1:
        out_f, in_f = getattr(module, "out_features", None), getattr(module, "in_features", None)
        if out_f is not None and in_f is not None and (
                m.numel() == out_f * in_f or (m.numel() < out_f * in_f and m.numel() % in_f == 0)):
            return (m.numel() // in_f, in_f) if in_f >= M else None
        return (1, m.numel()) if m.numel() >= M else None
    return None


@torch.no_grad()
def nm_2_4_tile_stats(model, debug=False):
    """Mean of the 2 larger and of the 2 smaller mask values of every group of 4 (:1029-1234)."""
    masks, tiles, n_sparse, skipped = [], 0.0, 0, []
    for name, module in _sparse_modules(model):
        n_sparse += 1
        m = module.mask.detach()
        view = _tile_view(module, m) if m.numel() > 0 else None
        if view is None:
            skipped.append((name, tuple(m.shape), m.dim()))
            continue
        r, c = view
        masks.append(m.reshape(r, c))
        tiles += float(r * (c // 4))
    if debug:
        print(f"[nm_2_4_tile_stats DEBUG] sparse_linear_count: {n_sparse}, processed: {len(masks)}, "
              f"total_tiles: {tiles}")
        if skipped:
            print(f"[nm_2_4_tile_stats DEBUG] skipped {len(skipped)} masks, first 3: {skipped[:3]}")
    if tiles <= 0:
        return {"top2_avg": 0.0, "bot2_avg": 0.0, "top2_gap": 0.0, "bot2_gap": 0.0, "total_gap": 0.0}
    rows = _mask_rows(masks)
    # per layer the reference sums in f32, then accumulates in f64
    top2_sum, bot2_sum = (float(rows[:, k].to(torch.float32).to(torch.float64).sum().item())
                          for k in (L.MSTAT_TOP2, L.MSTAT_BOT2))
    top2_avg = top2_sum / (tiles * 2)
    bot2_avg = bot2_sum / (tiles * 2)
    return {"top2_avg": top2_avg, "bot2_avg": bot2_avg, "top2_gap": 1.0 - top2_avg, "bot2_gap": bot2_avg,
            "total_gap": (1.0 - top2_avg) + bot2_avg}


@torch.no_grad()
def mask_stats(model, bins: int = 100, eps: float = 1e-8, sample_per_layer: int = 4096):
    """Global soft-mask statistics (:2069-2280): mean / std / entropy, threshold fractions, conditional
    means, histogram quantiles of sampled values and, for block_sparse layers, the lower / upper half
    means of the block means."""
    import math

    device = _model_device(model)
    mods = [m for _, m in _sparse_modules(model) if m.mask.numel() > 0]
    hist = torch.zeros((bins,), device=device, dtype=torch.int64)
    blk = torch.zeros(5, device=device, dtype=torch.float64)  # blocks, lower sum, lower count, upper sum, upper count
    if mods:
        masks = [m.mask.detach() for m in mods]
        rows = _mask_rows(masks, eps=eps)
        sums = rows.sum(dim=0).to(device)
        for mod, m in zip(mods, masks):
            take = min(m.numel(), int(sample_per_layer))
            if take > 0:
                idx = torch.randint(0, m.numel(), (take,), device=m.device)
                K.mask_hist(m.contiguous(), idx, bins, 0.0, 1.0, hist)
            hard_type = str(getattr(mod, "hard_mask_type", "match") or "match")
            if hard_type in ("block_sparse16", "block_sparse32") and m.dim() == 2:
                bs = 16 if hard_type == "block_sparse16" else 32
                if m.shape[0] >= bs and m.shape[1] >= bs:
                    means = K.block_stat(m.contiguous(), bs, L.BLOCK_MEAN)
                    nb = means.numel()
                    half = nb // 2
                    blk[0] += nb
                    if half > 0:
                        up_lo = K.keep_split_sum(means, K.topk_keep(means, nb - half)).to(device)
                        blk[1] += up_lo[1]
                        blk[2] += half
                        blk[3] += up_lo[0]
                        blk[4] += nb - half
    else:
        sums = torch.zeros(L.MSTAT_COUNT, device=device, dtype=torch.float64)
    tot = torch.tensor(float(sum(m.mask.numel() for m in mods)), device=device, dtype=torch.float64)
    hist64 = hist.to(torch.float64)
    _dist_sum(tot, sums, blk, hist64)
    tot_v = float(tot.item())
    if tot_v <= 0:
        return {"mask_mean": 1.0, "mask_std": 0.0, "mask_entropy": 0.0, "mask_hard_sparsity@0.5": 0.0,
                "mask_frac_lt_0.1": 0.0, "mask_frac_lt_0.01": 0.0, "mask_p10": 1.0, "mask_p50": 1.0,
                "mask_p90": 1.0}
    s = sums.cpu().tolist()
    mean = s[L.MSTAT_SUM] / tot_v
    std = math.sqrt(max(s[L.MSTAT_SUM2] / tot_v - mean * mean, 0.0))

    def frac(k):
        return s[k] / tot_v

    def q_from_hist(q: float) -> float:
        if float(hist64.sum().item()) <= 0:
            return mean
        cdf = (hist64.cumsum(0) / (hist64.sum() + 1e-12)).cpu()
        # q as a default (float32) tensor, as the reference passes it: 0.1f > 0.1 moves exact-0.1 CDF steps
        i = int(torch.searchsorted(cdf, torch.tensor([q])).item())
        return float((max(0, min(bins - 1, i)) + 0.5) / bins)

    b = blk.cpu().tolist()
    result = {
        "mask_mean": mean,
        "mask_std": std,
        "mask_entropy": s[L.MSTAT_ENTROPY] / tot_v,
        "mask_hard_sparsity@0.5": frac(L.MSTAT_LT05),
        "mask_frac_lt_0.1": frac(L.MSTAT_LT01),
        "mask_frac_lt_0.01": frac(L.MSTAT_LT001),
        "mask_frac_gt_0.9": frac(L.MSTAT_GT90),
        "mask_frac_gt_0.99": frac(L.MSTAT_GT99),
        "mask_frac_gt_0.5": frac(L.MSTAT_GT05),
        "mask_mean_lt_0.5": s[L.MSTAT_SUM_LT05] / s[L.MSTAT_LT05] if s[L.MSTAT_LT05] > 0 else 0.0,
        "mask_mean_gt_0.5": s[L.MSTAT_SUM_GT05] / s[L.MSTAT_GT05] if s[L.MSTAT_GT05] > 0 else 0.0,
        "mask_p10": q_from_hist(0.10),
        "mask_p50": q_from_hist(0.50),
        "mask_p90": q_from_hist(0.90),
    }
    if b[0] > 0:
        lower = b[1] / b[2] if b[2] > 0 else 0.0
        upper = b[3] / b[4] if b[4] > 0 else 0.0
        result["blk_lower_half_mean"] = lower
        result["blk_upper_half_mean"] = upper
        result["blk_total_blocks"] = b[0]
        result["blk_separation"] = upper - lower
    return result


@torch.no_grad()
def log_mask_stats(model, step: int, wandb_run=None, prefix: str = "mask/", bins: int = 100,
                   sample_per_layer: int = 4096):
    """mask_stats plus the schedule scalars of the first SparseLinear (:2283-2335), logged to
    `wandb_run` when one is given; returns the logged dict."""
    stats = mask_stats(model, bins=bins, sample_per_layer=sample_per_layer)
    log_dict = {prefix + k: v for k, v in stats.items()}
    log_dict["iter"] = step
    for _, module in _sparse_modules(model):
        log_dict[prefix + "beta_structural"] = float(module._beta_structural(step))
        log_dict[prefix + "hardening_x"] = float(getattr(module, "hardening_x", 1.0))
        break
    try:
        import torch.distributed as dist

        if dist.is_available() and dist.is_initialized() and dist.get_rank() != 0:
            return log_dict
    except Exception:
        pass
    if wandb_run is not None and hasattr(wandb_run, "log"):
        try:
            wandb_run.log(log_dict, step=step)
        except TypeError:
            wandb_run.log(log_dict)
    return log_dict


@torch.no_grad()
def harden_fraction(model, fraction: float = 0.2, band_low: float = 0.4, band_high: float = 0.6):
    """Round and freeze the `fraction` of unfrozen mask entries inside (band_low, band_high) that lie
    closest to 0.5, counted over all layers together (:1236-1276); returns how many were hardened.
    Every entry at the k-th smallest distance or closer is taken (ties included).  Off the paper
    path (hardening is 0 there): torch device ops, not a fused kernel."""
    layers = []
    for _, module in _sparse_modules(model):
        m = module.mask
        band = (m > band_low) & (m < band_high) & (module.frozen_mask_flags == 0)
        if bool(band.any()):
            layers.append((module, band, (m - 0.5).abs()))
    if not layers:
        return 0
    dists = torch.cat([d[b] for _, b, d in layers])
    k = int(dists.numel() * fraction)
    if k <= 0:
        return 0
    thr = torch.kthvalue(dists.float(), k).values.to(dists.dtype)
    hardened = 0
    for module, band, d in layers:
        pick = band & (d <= thr)
        module.mask.copy_(torch.where(pick, (module.mask > 0.5).to(module.mask.dtype), module.mask))
        module.frozen_mask_flags.copy_(torch.where(pick, torch.ones_like(module.frozen_mask_flags),
                                                   module.frozen_mask_flags))
        hardened += int(pick.sum())
    return hardened
