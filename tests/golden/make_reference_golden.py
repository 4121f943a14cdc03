"""Write golden input/output vectors of reference functions that no closed form pins.

Runs the reference code (liuhanzuo/SparseForge, /root/reference/legacy) in the
build container only, on small seeded inputs, and stores inputs and outputs
as .npz fixtures next to this script.  The fixtures are data; the reference
never travels with them.  Functions covered (reference file:line):

  gate_*      SparseLinear.compute_gate_target     legacy/sparse_modeling.py:1018-1239
  update_*    SparseLinear.update_mask (+ flips)   legacy/sparse_modeling.py:1242-1666
  glu_*       _update_glu_joint_mask               legacy/utils.py:363-479
  adamw_*     AdamW.step(decay=...)                legacy/adamw.py:65-176
  hutch_*     update_hessian_hutchinson            legacy/utils.py:714-869
  linear_*    FusedMaskedLinearSTE + SLoRB fwd/bwd legacy/sparse_modeling.py:56-132, :737-796
  ste_*       FusedMaskedLinearSTE.apply, decay    legacy/sparse_modeling.py:56-132
  kl_*        Distill_Model.kl_loss                legacy/sparse_modeling.py:1749-1828
  bsr_*       convert_to_block_sparse              legacy/triton_block_sparse.py:46-103
  hardblk_*   _hard_mask_from_soft, block types    legacy/sparse_modeling.py:537-718
  gateblk_*   compute_gate_target, block_sparse    legacy/sparse_modeling.py:1100-1158, :1237
  updblk_*    update_mask, block penalties/blockify legacy/sparse_modeling.py:1298-1529, :1598-1601
  stats_*     mid_penalty, sparsity_penalty,       legacy/utils.py:876-1234, :2069-2280
              nm_2_4_tile_stats, mask_stats
  harden_*    harden_fraction                      legacy/utils.py:1236-1276
  slorb_init_* init_SLoRB (projection P, weight S)  legacy/sparse_modeling.py:830-872
  *_obd_noH_* hessian_obd scores without a Hessian  legacy/sparse_modeling.py:1049-1055
              (compute_gate_target, update_mask)

The reference module imports wandb at top level without using it
(legacy/sparse_modeling.py:20); an empty module object is registered under
that name before the import.  The tau sample of _tau_unstructured draws
torch.randint right after torch.manual_seed(seed) inside compute_gate_target,
so the same indices are recorded by replaying that draw.

mask_stats samples torch.randint indices per layer; the draws are replayed
after the same torch.manual_seed and stored with the fixture.

Run:  python tests/golden/make_reference_golden.py [group ...]   (needs /root/reference;
      groups: gate update glu adamw hutch linear ste kl bsr block stats harden slorb, default all)
"""
from __future__ import annotations

import os
import sys
import types

import numpy as np
import torch

REF = os.environ.get("SF_REFERENCE_DIR", "/root/reference")
OUT = os.path.dirname(os.path.abspath(__file__))


def _import_reference():
    sys.modules.setdefault("wandb", types.ModuleType("wandb"))
    sys.path.insert(0, os.path.join(REF, "legacy"))
    import adamw as ref_adamw  # noqa: E402
    import sparse_modeling as ref_sm  # noqa: E402
    import utils as ref_utils  # noqa: E402

    return ref_sm, ref_utils, ref_adamw


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float32)


def make_layer(ref_sm, out_f, in_f, dtype, seed, no_hessian=False, **cfg_kw):
    cfg = ref_sm.SparseLinearConfig(**cfg_kw)
    if cfg_kw.get("mask_metric", "") in ("hessian_ratio", "hessian_obd", "hessian") and not no_hessian:
        cfg.enable_hutchinson = True
    torch.manual_seed(seed)
    layer = ref_sm.SparseLinear(in_f, out_f, sparselinear_config=cfg, bias=False).to(dtype)
    layer.weight.mask = layer.mask
    with torch.no_grad():
        layer.weight.copy_((torch.randn(out_f, in_f) * 0.02).to(dtype))
        if not layer._is_placeholder("hessian_diag"):
            layer.hessian_diag.copy_((torch.rand(out_f, in_f) * 1e-3 + 1e-5).to(dtype))
        layer.mask.copy_(torch.rand(out_f, in_f).to(dtype))
        if not layer._is_placeholder("frozen_mask_flags"):
            layer.frozen_mask_flags.copy_((torch.rand(out_f, in_f) < 0.05).to(dtype))
    return layer, cfg


def gate_cases(ref_sm, out):
    cases = {
        "gate_unstr_ratio_f32": dict(dtype=torch.float32, mask_type="unstructured", hard_mask_type="nm_2_4",
                                     mask_metric="hessian_ratio", tau_sample_size=512, sparsity_warmup_steps=100,
                                     step=40, beta_structural_start=0, beta_structural_end=0),
        "gate_unstr_beta_f32": dict(dtype=torch.float32, mask_type="unstructured", hard_mask_type="nm_2_4",
                                    mask_metric="hessian_obd", tau_sample_size=512, sparsity_warmup_steps=10,
                                    step=30, beta_structural_start=10, beta_structural_end=50),
        "gate_unstr_frozen_f32": dict(dtype=torch.float32, mask_type="unstructured", hard_mask_type="nm_2_4",
                                      mask_metric="magnitude", tau_sample_size=4096, sparsity_warmup_steps=0,
                                      step=7, freeze_low=0.05, freeze_high=0.95),
        "gate_struct_f32": dict(dtype=torch.float32, mask_type="structured", hard_mask_type="match",
                                mask_metric="hessian_ratio", tau_sample_size=512, step=25, temp_init=0.5),
        "gate_struct_exact_f32": dict(dtype=torch.float32, mask_type="structured", hard_mask_type="match",
                                      mask_metric="magnitude", structured_exact=True, step=3),
        "gate_unstr_ratio_bf16": dict(dtype=torch.bfloat16, mask_type="unstructured", hard_mask_type="nm_2_4",
                                      mask_metric="hessian_ratio", tau_sample_size=512, step=40),
        "gate_struct_bf16": dict(dtype=torch.bfloat16, mask_type="structured", hard_mask_type="match",
                                 mask_metric="hessian_obd", step=12, beta_structural_start=0,
                                 beta_structural_end=20),
        # hessian_diag left a placeholder: the score falls back to W * W (:1053-1055)
        "gate_obd_noH_f32": dict(dtype=torch.float32, mask_type="unstructured", hard_mask_type="nm_2_4",
                                 mask_metric="hessian_obd", tau_sample_size=512, sparsity_warmup_steps=0,
                                 step=9, no_hessian=True),
        "gate_obd_noH_bf16": dict(dtype=torch.bfloat16, mask_type="structured", hard_mask_type="match",
                                  mask_metric="hessian_obd", step=4, no_hessian=True),
    }
    for i, (name, kw) in enumerate(cases.items()):
        kw = dict(kw)
        dtype = kw.pop("dtype")
        step = kw.pop("step")
        layer, cfg = make_layer(ref_sm, 32, 64, dtype, 100 + i, **kw)
        kw.pop("no_hessian", None)
        seed = 1000 + i
        torch.manual_seed(seed)
        G = layer.compute_gate_target(step)
        n = layer.weight.numel()
        m = int(cfg.tau_sample_size)
        torch.manual_seed(seed)
        idx = torch.randint(0, n, (m,)) if (m > 0 and n > m) else torch.arange(n)
        out[name] = dict(W=np32(layer.weight), H=np32(layer.hessian_diag), mask=np32(layer.mask),
                         frozen=np32(layer.frozen_mask_flags), idx=idx.numpy().astype(np.int64), G=np32(G),
                         step=np.int64(step), T=np.float64(layer._temperature(step)),
                         sparsity=np.float64(layer._effective_sparsity(step)),
                         beta_s=np.float64(layer._beta_structural(step)),
                         dtype=np.array(str(dtype)), cfg=np.array(repr(kw)))


def update_cases(ref_sm, out):
    cases = {
        "update_paper_f32": dict(dtype=torch.float32, mask_type="unstructured", hard_mask_type="nm_2_4",
                                 mask_metric="hessian_ratio", tau_sample_size=512, sparsity_warmup_steps=0,
                                 mask_update_period=1, mask_penalty_mode="nm_2_4", mask_penalty_lr=0.1,
                                 mask_lr=0.1, mask_hardening_start=3, mask_hardening_duration=4, lam=0.1),
        "update_mid_bin_f32": dict(dtype=torch.float32, mask_type="unstructured", hard_mask_type="match",
                                   mask_metric="magnitude", tau_sample_size=512, sparsity_warmup_steps=0,
                                   mask_update_period=1, mask_penalty_mode="mid", mask_binarize_decay=0.05,
                                   mask_lr=0.2, lam=0.3),
        "update_struct_topn_f32": dict(dtype=torch.float32, mask_type="structured", hard_mask_type="match",
                                       mask_metric="hessian_obd", sparsity_warmup_steps=0, mask_update_period=1,
                                       mask_penalty_mode="structured_topn", mask_lr=0.15, lam=0.2,
                                       beta_structural_start=0, beta_structural_end=6),
        "update_freeze_f32": dict(dtype=torch.float32, mask_type="unstructured", hard_mask_type="nm_2_4",
                                  mask_metric="magnitude", tau_sample_size=100000, sparsity_warmup_steps=0,
                                  mask_update_period=1, freeze_low=0.2, freeze_high=0.8, mask_lr=0.3, lam=0.0,
                                  steps=(1998, 1999, 2000, 2001)),
        "update_paper_bf16": dict(dtype=torch.bfloat16, mask_type="unstructured", hard_mask_type="nm_2_4",
                                  mask_metric="hessian_ratio", tau_sample_size=512, sparsity_warmup_steps=0,
                                  mask_update_period=1, mask_penalty_mode="nm_2_4", mask_penalty_lr=0.1,
                                  mask_lr=0.1, lam=0.1),
        "update_obd_noH_f32": dict(dtype=torch.float32, mask_type="unstructured", hard_mask_type="nm_2_4",
                                   mask_metric="hessian_obd", tau_sample_size=512, sparsity_warmup_steps=0,
                                   mask_update_period=1, mask_penalty_mode="nm_2_4", mask_penalty_lr=0.1,
                                   mask_lr=0.1, lam=0.1, steps=(1, 2, 3), no_hessian=True),
    }
    for i, (name, kw) in enumerate(cases.items()):
        kw = dict(kw)
        dtype = kw.pop("dtype")
        lam = kw.pop("lam")
        steps = kw.pop("steps", (1, 2, 3, 4, 5))
        # 32 x 66: a 2-column tail after 16 full groups (nm_2_4 keeps the tail)
        cols = 64 if kw["mask_type"] == "structured" else 66
        kw_rec = {k: v for k, v in kw.items() if k != "no_hessian"}
        layer, cfg = make_layer(ref_sm, 32, cols, dtype, 200 + i, **kw)
        rec = dict(W=np32(layer.weight), H=np32(layer.hessian_diag), init_mask=np32(layer.mask),
                   init_frozen=np32(layer.frozen_mask_flags), dtype=np.array(str(dtype)), cfg=np.array(repr(kw_rec)),
                   lam=np.float64(lam), steps=np.array(steps, dtype=np.int64))
        n = layer.weight.numel()
        m = int(cfg.tau_sample_size)
        for j, step in enumerate(steps):
            seed = 5000 + 10 * i + j
            torch.manual_seed(seed)
            idx = torch.randint(0, n, (m,)) if (m > 0 and n > m) else torch.arange(n)
            torch.manual_seed(seed)
            layer.update_mask(step, lambda_mid=lam)
            rec[f"idx{j}"] = idx.numpy().astype(np.int64)
            rec[f"mask{j}"] = np32(layer.mask)
            rec[f"frozen{j}"] = np32(layer.frozen_mask_flags)
            rec[f"flips{j}"] = np.int64(layer.weight.flipped_mask)
            rec[f"hx{j}"] = np.float64(layer.hardening_x)
            rec[f"T{j}"] = np.float64(layer._temperature(step))
            rec[f"sparsity{j}"] = np.float64(layer._effective_sparsity(step))
            rec[f"beta{j}"] = np.float64(layer._beta_structural(step))
        out[name] = rec


def glu_case(ref_sm, ref_utils, out):
    kw = dict(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio", tau_sample_size=512,
              sparsity_warmup_steps=0, mask_update_period=1, mask_penalty_mode="mid", mask_lr=0.1,
              glu_joint_mask=True, mask_hardening_start=2, mask_hardening_duration=10)
    gate, cfg = make_layer(ref_sm, 32, 64, torch.float32, 300, **kw)
    up, _ = make_layer(ref_sm, 32, 64, torch.float32, 301, **kw)
    rec = dict(Wg=np32(gate.weight), Hg=np32(gate.hessian_diag), init_Mg=np32(gate.mask), Wu=np32(up.weight),
               Hu=np32(up.hessian_diag), init_Mu=np32(up.mask), cfg=np.array(repr(kw)))
    n = gate.weight.numel()
    for j, step in enumerate((1, 2, 3)):
        seed = 7000 + j
        torch.manual_seed(seed)
        idx = torch.randint(0, n, (512,))
        torch.manual_seed(seed)
        ref_utils._update_glu_joint_mask(gate, up, step, 0.05)
        rec[f"idx{j}"] = idx.numpy().astype(np.int64)
        rec[f"Mg{j}"] = np32(gate.mask)
        rec[f"Mu{j}"] = np32(up.mask)
        rec[f"flips_g{j}"] = np.int64(gate.weight.flipped_mask)
        rec[f"flips_u{j}"] = np.int64(up.weight.flipped_mask)
        rec[f"hx{j}"] = np.float64(gate.hardening_x)
    out["glu_joint_f32"] = rec


def adamw_cases(ref_adamw, out):
    cases = {
        "adamw_decay_l1": dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, amsgrad=False,
                               srste_decay=2e-4, adaptive_l1_decay=1e-3, decays=(None, 3e-4, 5e-4, 0.0)),
        "adamw_amsgrad": dict(lr=2e-3, betas=(0.8, 0.99), eps=1e-6, weight_decay=0.0, amsgrad=True,
                              srste_decay=None, adaptive_l1_decay=0.0, decays=(1e-3, 1e-3, 1e-3)),
        "adamw_plain": dict(lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2, amsgrad=False,
                            srste_decay=None, adaptive_l1_decay=0.0, decays=(None, None, None)),
    }
    for i, (name, kw) in enumerate(cases.items()):
        kw = dict(kw)
        decays = kw.pop("decays")
        g = torch.Generator().manual_seed(400 + i)
        w = torch.nn.Parameter(torch.randn(24, 40, generator=g) * 0.05)
        w.mask = torch.rand(24, 40, generator=g)
        b = torch.nn.Parameter(torch.randn(40, generator=g) * 0.05)  # no mask, 1-D
        opt = ref_adamw.AdamW([w, b], **kw)
        rec = dict(init_w=np32(w), init_b=np32(b), mask=np32(w.mask), cfg=np.array(repr(kw)))
        for j, d in enumerate(decays):
            w.grad = torch.randn(24, 40, generator=g) * 1e-2
            b.grad = torch.randn(40, generator=g) * 1e-2
            rec[f"gw{j}"] = np32(w.grad)
            rec[f"gb{j}"] = np32(b.grad)
            opt.step(decay=d)
            rec[f"w{j}"] = np32(w)
            rec[f"b{j}"] = np32(b)
            st = opt.state[w]
            rec[f"m{j}"] = np32(st["exp_avg"])
            rec[f"v{j}"] = np32(st["exp_avg_sq"])
            if kw["amsgrad"]:
                rec[f"vmax{j}"] = np32(st["max_exp_avg_sq"])
            rec[f"decay{j}"] = np.float64(opt.decay)
        out[name] = rec


def hutchinson_case(ref_sm, ref_utils, out):
    kw = dict(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio", beta=0.98)
    layer, cfg = make_layer(ref_sm, 24, 48, torch.float32, 500, **kw)
    torch.manual_seed(501)
    x = torch.randn(64, 48)
    y = torch.randn(64, 24)
    rec = dict(W=np32(layer.weight), mask=np32(layer.mask), init_H=np32(layer.hessian_diag), x=np32(x), y=np32(y))
    for j in range(3):
        out_ = layer(x)
        loss = 0.5 * ((out_ - y) ** 2).sum()
        torch.manual_seed(600 + j)
        v = (torch.randint_like(layer.weight, low=0, high=2, dtype=torch.int8).float() * 2 - 1)
        torch.manual_seed(600 + j)
        ref_utils.update_hessian_hutchinson(layer, loss)
        rec[f"v{j}"] = np32(v)
        rec[f"H{j}"] = np32(layer.hessian_diag)
        layer.zero_grad(set_to_none=True)
    out["hutch_quadratic_f32"] = rec


def linear_case(ref_sm, out):
    kw = dict(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio", SLoRB=True,
              SLoRB_k=8, SLoRB_init_type="sum", trainable_projection=True, weight_scaling=True)
    cfg = ref_sm.SparseLinearConfig(**kw)
    torch.manual_seed(700)
    layer = ref_sm.SparseLinear(32, 20, sparselinear_config=cfg, bias=True)
    with torch.no_grad():
        layer.weight.copy_(torch.randn(20, 32) * 0.02)
        layer.bias.copy_(torch.randn(20) * 0.1)
        layer.mask.copy_(torch.rand(20, 32))
        layer.init_SLoRB()
        layer.SLoRB_Weight.copy_(torch.randn(20, 4) * 0.01)
    rec = dict(W=np32(layer.weight), bias=np32(layer.bias), mask=np32(layer.mask), P=np32(layer.x_proj),
               S=np32(layer.SLoRB_Weight), cfg=np.array(repr(kw)))
    for j, hx in enumerate((1.0, 0.4, 0.0)):
        layer.hardening_x = hx
        x = torch.randn(3, 5, 32, requires_grad=True)
        y = layer(x)
        gy = torch.randn_like(y)
        y.backward(gy)
        rec[f"hx{j}"] = np.float64(hx)
        rec[f"x{j}"] = np32(x)
        rec[f"y{j}"] = np32(y)
        rec[f"gy{j}"] = np32(gy)
        rec[f"dx{j}"] = np32(x.grad)
        rec[f"dW{j}"] = np32(layer.weight.grad)
        rec[f"db{j}"] = np32(layer.bias.grad)
        rec[f"dP{j}"] = np32(layer.x_proj.grad)
        rec[f"dS{j}"] = np32(layer.SLoRB_Weight.grad)
        layer.zero_grad(set_to_none=True)
    out["linear_slorb_f32"] = rec


def slorb_init_cases(ref_sm, out):
    """init_SLoRB on a layer with a random soft mask: the block-sum projection P and the SLoRB weight S
    (the sum or mean of the pruned part W (1 - mask) over each block of k inputs)."""
    for name, (out_f, in_f, k, init, dtype) in {"slorb_init_sum_f32": (20, 32, 8, "sum", torch.float32),
                                                  "slorb_init_mean_f32": (24, 48, 16, "mean", torch.float32),
                                                  "slorb_init_mean_bf16": (16, 64, 8, "mean", torch.bfloat16)}.items():
        kw = dict(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="magnitude", SLoRB=True,
                  SLoRB_k=k, SLoRB_init_type=init, trainable_projection=True)
        cfg = ref_sm.SparseLinearConfig(**kw)
        torch.manual_seed(750 + k)
        layer = ref_sm.SparseLinear(in_f, out_f, sparselinear_config=cfg, bias=False).to(dtype)
        with torch.no_grad():
            layer.weight.copy_((torch.randn(out_f, in_f) * 0.02).to(dtype))
            layer.mask.copy_(torch.rand(out_f, in_f).to(dtype))
        layer.init_SLoRB()
        out[name] = dict(W=np32(layer.weight), mask=np32(layer.mask), P=np32(layer.x_proj),
                         S=np32(layer.SLoRB_Weight), dtype=np.array(str(dtype)), cfg=np.array(repr(kw)))


def ste_cases(ref_sm, out):
    """FusedMaskedLinearSTE.apply(x, W, b, mask, decay, scale) with decay != 0 and scale != 1
    (:56-132): forward, backward (dW carries decay * W * [mask < 0.5]) and the Hessian-vector
    product of a quadratic loss by double backward (the decay term is differentiated too)."""
    for dt, tag in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
        torch.manual_seed(720)
        x = torch.randn(2, 40, 64).to(dt)
        W = (torch.randn(48, 64) * 0.02).to(dt)
        b = (torch.randn(48) * 0.1).to(dt)
        mask = torch.rand(48, 64)
        mask[:, ::7] = 0.5  # entries exactly at the decay threshold (kept: the test is mask < 0.5)
        gy = torch.randn(2, 40, 48).to(dt)
        t = torch.randn(2, 40, 48).to(dt)
        v = (torch.randint(0, 2, (48, 64)) * 2 - 1).to(dt)
        decay, scale = 0.05, 1.7
        xr, Wr, br = x.clone().requires_grad_(True), W.clone().requires_grad_(True), b.clone().requires_grad_(True)
        y = ref_sm.FusedMaskedLinearSTE.apply(xr, Wr, br, mask, decay, scale)
        y.backward(gy)
        rec = dict(x=np32(x), W=np32(W), b=np32(b), mask=np32(mask), gy=np32(gy), t=np32(t), v=np32(v),
                   decay=np.float64(decay), scale=np.float64(scale), y=np32(y), dx=np32(xr.grad),
                   dW=np32(Wr.grad), db=np32(br.grad))
        Wh = W.clone().requires_grad_(True)
        yh = ref_sm.FusedMaskedLinearSTE.apply(x, Wh, b, mask, decay, scale)
        loss = 0.5 * ((yh.float() - t.float()) ** 2).sum()
        (g,) = torch.autograd.grad(loss, Wh, create_graph=True)
        (hvp,) = torch.autograd.grad((g * v).sum(), Wh)
        rec["hvp"] = np32(hvp)
        out[f"ste_decay_{tag}"] = rec


def kl_case(ref_sm, out):
    torch.manual_seed(800)
    s = torch.randn(2, 37, 300) * 4
    t = torch.randn(2, 37, 300) * 4
    s[0, 3, 7] = 250.0  # exercises the +-100 clamp
    t[1, 5, 9] = -400.0
    d = ref_sm.Distill_Model.__new__(ref_sm.Distill_Model)
    # kl_loss clamps and scales float32 logits in place (.float() aliases them, :1788-1796):
    # it gets copies, and the copies are recorded after the call as s_after / t_after
    s_in, t_in = s.clone(), t.clone()
    kl = ref_sm.Distill_Model.kl_loss(d, s_in, t_in)
    out["kl_basic_f32"] = dict(s=np32(s), t=np32(t), kl=np.float64(kl.item()), s_after=np32(s_in),
                               t_after=np32(t_in))


def bsr_case(out):
    sys.path.insert(0, os.path.join(REF, "legacy"))
    import triton_block_sparse as ref_bs  # noqa: E402

    g = torch.Generator().manual_seed(1)
    W = torch.randn(64, 96, generator=g) * 0.02
    bm = (torch.rand(4, 6, generator=g) < 0.5).float()
    mask = bm.repeat_interleave(16, 0).repeat_interleave(16, 1)
    mask[0:16, 16:32] = 0.0  # fully pruned block
    mask[16, 48] = 0.0       # a zero inside an otherwise kept block
    W[32:48, 0:16] = 0.0     # a kept-by-mask block whose weights are all zero (dropped: nonzero test uses W*M)
    blocks, row_ptr, col_idx = ref_bs.convert_to_block_sparse(W, mask, 16)
    out["bsr_basic_f32"] = dict(W=np32(W), mask=np32(mask), blocks=np32(blocks), row_ptr=row_ptr.numpy(),
                                col_idx=col_idx.numpy())


def block_cases(ref_sm, out):
    """Block hard types, the block_sparse gate and the block penalty modes on ragged shapes
    (edges outside the fully covered core) with distinct random values, plus all-equal inputs
    (the tie case whose torch.topk order is fixed: the higher index wins)."""
    hard = {
        "hardblk_block16_f32": ("block16", (40, 56), 0.5, "rand"),
        "hardblk_block16_sr03_f32": ("block16", (40, 56), 0.3, "rand"),
        "hardblk_block16_ones_f32": ("block16", (16, 32), 0.5, "ones"),
        "hardblk_bs16_f32": ("block_sparse16", (72, 100), 0.5, "rand"),
        "hardblk_bs16_sr03_f32": ("block_sparse16", (72, 100), 0.3, "rand"),
        "hardblk_bs16_ones_f32": ("block_sparse16", (64, 64), 0.5, "ones"),
        "hardblk_bs32_f32": ("block_sparse32", (100, 70), 0.5, "rand"),
    }
    for i, (name, (ht, shape, sr, kind)) in enumerate(hard.items()):
        layer, _ = make_layer(ref_sm, shape[0], shape[1], torch.float32, 900 + i, mask_type="unstructured",
                              hard_mask_type=ht, sparsity_ratio=sr)
        g = torch.Generator().manual_seed(950 + i)
        soft = torch.rand(shape, generator=g) if kind == "rand" else torch.ones(shape)
        hard_ = layer._hard_mask_from_soft(soft)
        out[name] = dict(soft=np32(soft), hard=np32(hard_), hard_type=np.array(ht), sr=np.float64(sr))

    gates = {
        "gateblk_bs16_f32": dict(shape=(40, 72), mask_type="unstructured", hard_mask_type="block_sparse16",
                                 mask_metric="hessian_ratio", tau_sample_size=512, sparsity_warmup_steps=100,
                                 step=60, freeze_low=0.05),
        "gateblk_bs32_struct_f32": dict(shape=(64, 96), mask_type="structured", hard_mask_type="block_sparse32",
                                        mask_metric="magnitude", step=9, beta_structural_start=0,
                                        beta_structural_end=20),
        "gateblk_bs16_small_f32": dict(shape=(12, 40), mask_type="unstructured", hard_mask_type="block_sparse16",
                                       mask_metric="magnitude", tau_sample_size=100, step=5),
    }
    for i, (name, kw) in enumerate(gates.items()):
        kw = dict(kw)
        shape, step = kw.pop("shape"), kw.pop("step")
        layer, cfg = make_layer(ref_sm, shape[0], shape[1], torch.float32, 920 + i, **kw)
        seed = 9200 + i
        torch.manual_seed(seed)
        G = layer.compute_gate_target(step)
        n = layer.weight.numel()
        m = int(cfg.tau_sample_size)
        torch.manual_seed(seed)
        idx = torch.randint(0, n, (m,)) if (m > 0 and n > m) else torch.arange(n)
        out[name] = dict(W=np32(layer.weight), H=np32(layer.hessian_diag), mask=np32(layer.mask),
                         frozen=np32(layer.frozen_mask_flags), idx=idx.numpy().astype(np.int64), G=np32(G),
                         step=np.int64(step), T=np.float64(layer._temperature(step)),
                         sparsity=np.float64(layer._effective_sparsity(step)), dtype=np.array(str(torch.float32)),
                         cfg=np.array(repr(kw)))

    updates = {
        "updblk_bs16_f32": dict(shape=(50, 84), mask_type="unstructured", hard_mask_type="block_sparse16",
                                mask_metric="hessian_ratio", tau_sample_size=512, sparsity_warmup_steps=0,
                                mask_update_period=1, mask_penalty_mode="block_sparse16", mask_penalty_lr=0.1,
                                mask_binarize_decay=0.05, mask_lr=0.2, lam=0.2),
        "updblk_block16_pen_f32": dict(shape=(36, 50), mask_type="unstructured", hard_mask_type="nm_2_4",
                                       mask_metric="magnitude", tau_sample_size=512, sparsity_warmup_steps=0,
                                       mask_update_period=1, mask_penalty_mode="block16", mask_penalty_lr=0.2,
                                       mask_lr=0.15, lam=0.3),
        "updblk_bs32_freeze_f32": dict(shape=(64, 70), mask_type="unstructured", hard_mask_type="block_sparse32",
                                       mask_metric="magnitude", tau_sample_size=100000, sparsity_warmup_steps=0,
                                       mask_update_period=1, mask_penalty_mode="mid", freeze_low=0.3,
                                       freeze_high=0.7, mask_lr=0.4, lam=0.1, steps=(1999, 2000, 2001)),
        "updblk_block16_hard_f32": dict(shape=(32, 48), mask_type="structured", hard_mask_type="block16",
                                        mask_metric="hessian_obd", sparsity_warmup_steps=0, mask_update_period=1,
                                        mask_penalty_mode="block_sparse32", mask_lr=0.2, lam=0.2),
    }
    for i, (name, kw) in enumerate(updates.items()):
        kw = dict(kw)
        shape, lam = kw.pop("shape"), kw.pop("lam")
        steps = kw.pop("steps", (1, 2, 3, 4))
        layer, cfg = make_layer(ref_sm, shape[0], shape[1], torch.float32, 940 + i, **kw)
        rec = dict(W=np32(layer.weight), H=np32(layer.hessian_diag), init_mask=np32(layer.mask),
                   init_frozen=np32(layer.frozen_mask_flags), dtype=np.array(str(torch.float32)),
                   cfg=np.array(repr(kw)), lam=np.float64(lam), steps=np.array(steps, dtype=np.int64))
        n = layer.weight.numel()
        m = int(cfg.tau_sample_size)
        for j, step in enumerate(steps):
            seed = 9400 + 10 * i + j
            torch.manual_seed(seed)
            idx = torch.randint(0, n, (m,)) if (m > 0 and n > m) else torch.arange(n)
            torch.manual_seed(seed)
            layer.update_mask(step, lambda_mid=lam)
            rec[f"idx{j}"] = idx.numpy().astype(np.int64)
            rec[f"mask{j}"] = np32(layer.mask)
            rec[f"frozen{j}"] = np32(layer.frozen_mask_flags)
            rec[f"flips{j}"] = np.int64(layer.weight.flipped_mask)
            rec[f"hx{j}"] = np.float64(layer.hardening_x)
        out[name] = rec


def _bf16_neighbours(vals):
    """bf16 values at and one bf16 step either side of each value."""
    b = torch.tensor(vals, dtype=torch.float32).bfloat16()
    bits = b.view(torch.int16)
    out = [b, (bits + 1).view(torch.bfloat16), (bits - 1).view(torch.bfloat16)]
    return torch.cat(out).float()


def stats_cases(ref_sm, ref_utils, out):
    """Penalties and mask statistics over small models of several SparseLinear layers: f32 and
    bf16 masks, a ragged tail (in % 4 != 0), structured / unstructured / block_sparse types,
    values on and next to the thresholds, and a layer holding NaN and an exact 1."""
    specials = [0.0, 1e-9, 0.01, 0.1, 0.5, 0.9, 0.99, 0.999999]
    models = {
        "stats_f32": (torch.float32, [((24, 36), "structured", "nm_2_4"), ((20, 30), "unstructured", "nm_2_4"),
                                      ((32, 48), "unstructured", "block_sparse16"),
                                      ((10, 30), "structured", "nm_2_4")], "specials"),
        "stats_bf16": (torch.bfloat16, [((16, 40), "structured", "nm_2_4"),
                                        ((64, 40), "unstructured", "block_sparse32"),
                                        ((12, 22), "structured", "nm_2_4")], "bf16edges"),
        "stats_nan_f32": (torch.float32, [((8, 16), "structured", "nm_2_4"), ((8, 12), "unstructured", "nm_2_4")],
                          "nan"),
    }
    for mi, (name, (dtype, layers, kind)) in enumerate(models.items()):
        model = torch.nn.Module()
        g = torch.Generator().manual_seed(1200 + mi)
        rec = {}
        for li, ((o, i), mt, ht) in enumerate(layers):
            layer, _ = make_layer(ref_sm, o, i, dtype, 1300 + 10 * mi + li, mask_type=mt, hard_mask_type=ht)
            m = torch.rand(o, i, generator=g)
            if li == 1 and kind == "specials":
                m.view(-1)[: len(specials)] = torch.tensor(specials)
            if li == 0 and kind == "bf16edges":
                e = _bf16_neighbours([0.01, 0.1, 0.5, 0.9, 0.99])
                m.view(-1)[: e.numel()] = e
            if li == 0 and kind == "nan":
                m[0, 1] = float("nan")
                m[3, 2] = 1.0
            with torch.no_grad():
                layer.mask.copy_(m.to(dtype))
            model.add_module(f"l{li}", layer)
            rec[f"mask{li}"] = np32(layer.mask)
            rec[f"mask_type{li}"] = np.array(mt)
            rec[f"hard_type{li}"] = np.array(ht)
        rec["dtype"] = np.array("bf16" if dtype == torch.bfloat16 else "f32")
        rec["n_layers"] = np.int64(len(layers))
        rec["mid"] = np.float64(ref_utils.mid_penalty(model, 0.7).item())
        pen, cur = ref_utils.sparsity_penalty(model, 0.4, 2.0)
        rec["sp_pen"], rec["sp_cur"] = np.float64(pen.item()), np.float64(cur)
        ts = ref_utils.nm_2_4_tile_stats(model)
        rec["tile_keys"] = np.array(sorted(ts))
        rec["tile_vals"] = np.array([ts[k] for k in sorted(ts)], dtype=np.float64)
        seed, sample = 1400 + mi, 300
        torch.manual_seed(seed)
        ms = ref_utils.mask_stats(model, bins=100, sample_per_layer=sample)
        rec["ms_keys"] = np.array(sorted(ms))
        rec["ms_vals"] = np.array([ms[k] for k in sorted(ms)], dtype=np.float64)
        torch.manual_seed(seed)  # replay the per-layer sample draws of mask_stats (:2145-2148)
        for li, ((o, i), _, _) in enumerate(layers):
            rec[f"idx{li}"] = torch.randint(0, o * i, (min(o * i, sample),)).numpy()
        rec["sample"] = np.int64(sample)
        out[name] = rec


def harden_case(ref_sm, ref_utils, out):
    """harden_fraction over two layers with real frozen flags: masks spread around 0.5 (some on the
    band edges, some already frozen, repeated values at the threshold)."""
    model = torch.nn.Module()
    g = torch.Generator().manual_seed(1500)
    rec = {}
    for li, (o, i) in enumerate([(16, 24), (8, 40)]):
        layer, _ = make_layer(ref_sm, o, i, torch.float32, 1510 + li, mask_type="unstructured",
                              hard_mask_type="nm_2_4", freeze_low=0.05, freeze_high=0.95)
        m = 0.3 + 0.4 * torch.rand(o, i, generator=g)
        m.view(-1)[:6] = torch.tensor([0.4, 0.6, 0.5, 0.5, 0.45, 0.55])
        fz = (torch.rand(o, i, generator=g) < 0.1).float()
        with torch.no_grad():
            layer.mask.copy_(m)
            layer.frozen_mask_flags.copy_(fz)
        model.add_module(f"l{li}", layer)
        rec[f"mask_in{li}"] = np32(layer.mask)
        rec[f"frozen_in{li}"] = np32(layer.frozen_mask_flags)
    rec["count"] = np.int64(ref_utils.harden_fraction(model, 0.2, 0.4, 0.6))
    for li, layer in enumerate(model.children()):
        rec[f"mask_out{li}"] = np32(layer.mask)
        rec[f"frozen_out{li}"] = np32(layer.frozen_mask_flags)
    out["harden_f32"] = rec


GROUPS = ("gate", "update", "glu", "adamw", "hutch", "linear", "ste", "kl", "bsr", "block", "stats", "harden",
          "slorb")


def main():
    ref_sm, ref_utils, ref_adamw = _import_reference()
    torch.set_num_threads(1)
    groups = set(sys.argv[1:]) or set(GROUPS)
    unknown = groups - set(GROUPS)
    if unknown:
        raise SystemExit(f"unknown groups {sorted(unknown)}; known: {GROUPS}")
    out = {}
    if "gate" in groups:
        gate_cases(ref_sm, out)
    if "update" in groups:
        update_cases(ref_sm, out)
    if "glu" in groups:
        glu_case(ref_sm, ref_utils, out)
    if "adamw" in groups:
        adamw_cases(ref_adamw, out)
    if "hutch" in groups:
        hutchinson_case(ref_sm, ref_utils, out)
    if "linear" in groups:
        linear_case(ref_sm, out)
    if "kl" in groups:
        kl_case(ref_sm, out)
    if "ste" in groups:
        ste_cases(ref_sm, out)
    if "bsr" in groups:
        bsr_case(out)
    if "block" in groups:
        block_cases(ref_sm, out)
    if "stats" in groups:
        stats_cases(ref_sm, ref_utils, out)
    if "harden" in groups:
        harden_case(ref_sm, ref_utils, out)
    if "slorb" in groups:
        slorb_init_cases(ref_sm, out)
    for name, rec in out.items():
        path = os.path.join(OUT, f"ref_{name}.npz")
        np.savez_compressed(path, torch_version=np.array(torch.__version__), **rec)
    total = sum(os.path.getsize(os.path.join(OUT, f"ref_{n}.npz")) for n in out)
    print(f"wrote {len(out)} fixtures, {total / 1024:.1f} KiB")


if __name__ == "__main__":
    main()
