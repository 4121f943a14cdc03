"""One full sparse retraining step on the GPU against the float64 CPU restatement (oracle/retrain.py).

A 2-layer, hidden-128 LLaMA-architecture student (every projection a
SparseLinear, unstructured soft mask with a hard 2:4 projection, SLoRB rank
64, hessian_ratio scores with Hutchinson) distils from a dense teacher over 2
micro-batches; the step follows legacy/main_llama.py:1996-2211.  Two steps
run (iteration 1 with the mixed hardening mask, iteration 2 after the first
mask update); each step starts the oracle from the GPU's own state.

Bars (float32 model, the north-star float32 tolerances):
* loss, clipped gradients of every trainable parameter and the Hutchinson
  accumulator: within 1e-5 of the float64 restatement, relative to each
  tensor's largest magnitude;
* AdamW: the GPU's updated parameters and moments equal oracle.adamw.step on
  the GPU's own pre-step parameters and clipped gradients bit for bit;
* mask update: the GPU's new soft masks within 1e-6 of
  oracle.masks.layer_update_mask on the GPU's own post-step W and H, hard 2:4
  projections equal, flip counts equal;
* end to end (the oracle's own chain): parameters with a clear gradient
  within 1e-5 (Adam's normalised step is ill-conditioned where the gradient
  is near zero: those entries within two learning-rate steps), soft masks
  within 1e-5 for 99% of the entries and within one EMA step everywhere.
"""
import itertools

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

RANK = 64


def _shape():
    from sparseforge_amd.llama import LlamaShape

    return LlamaShape(vocab_size=512, hidden_size=128, intermediate_size=384, num_hidden_layers=2,
                      num_attention_heads=4)


CFG = dict(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio", beta=0.98,
           mask_update_period=1, sparsity_warmup_steps=0, mask_hardening_start=0, mask_hardening_duration=4,
           mask_penalty_mode="nm_2_4", mask_penalty_lr=0.1, mask_lr=0.1, tau_sample_size=262144, SLoRB=True,
           SLoRB_init_type="sum", trainable_projection=True)
STEP = dict(grad_accum=2, hardness_task=1.0, hardness_kldiv=1.0, lambda_mid_max=0.1, sparsity_ratio=0.5,
            sparsity_alpha=0.2, grad_clip=1.0, hutchinson=True, mask_penalty_mode="nm_2_4", lr=1e-3, decay=0.0,
            betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _build(dev):
    from sparseforge_amd import sparse_modeling as sm
    from sparseforge_amd.adamw import AdamW
    from sparseforge_amd.llama import LlamaDecoder
    from sparseforge_amd.retrain import RetrainConfig, optimizer_groups

    shape = _shape()
    cfg = sm.SparseLinearConfig(**CFG)
    cfg.enable_hutchinson = True
    g = torch.Generator(device=dev).manual_seed(3)
    student = LlamaDecoder(shape, cfg, RANK, dev, torch.float32)
    student.init_random(g)
    teacher = LlamaDecoder(shape, None, RANK, dev, torch.float32)
    teacher.init_random(g)
    teacher.requires_grad_(False)
    with torch.no_grad():  # a mid-training state: soft masks, a Hessian accumulator, hardening under way
        for m in student.modules():
            if isinstance(m, sm.SparseLinear):
                m.mask.copy_(torch.rand(m.mask.shape, generator=g, device=dev))
                m.hessian_diag.copy_(torch.rand(m.mask.shape, generator=g, device=dev) * 1e-3 + 1e-6)
                m.hardening_x = 0.75
    opt = AdamW(optimizer_groups(student, STEP["weight_decay"]), lr=STEP["lr"], betas=STEP["betas"], eps=STEP["eps"])
    rc = RetrainConfig(**{k: v for k, v in STEP.items() if k not in ("betas", "eps", "weight_decay")},
                       autocast_dtype=None)
    return shape, student, teacher, opt, rc


def _snapshot(student, opt):
    from sparseforge_amd import sparse_modeling as sm

    st = {}
    for name, p in student.named_parameters():
        if name.endswith((".mask", ".hessian_diag", ".frozen_mask_flags", ".grad_ema", ".scaler_row")):
            continue
        st[name] = p.detach().float().cpu().numpy().copy()
        s = opt.state.get(p, {})
        if s:
            st[name + ".exp_avg"] = s["exp_avg"].cpu().numpy().copy()
            st[name + ".exp_avg_sq"] = s["exp_avg_sq"].cpu().numpy().copy()
            st[name + ".step"] = int(s["step"])
    for name, m in student.named_modules():
        if isinstance(m, sm.SparseLinear):
            st[name + ".mask"] = m.mask.detach().cpu().numpy().copy()
            st[name + ".hessian_diag"] = m.hessian_diag.detach().cpu().numpy().copy()
            st[name + ".hx"] = float(m.hardening_x)
    return st


def test_retrain_step_matches_float64_restatement(cuda_device, monkeypatch):
    from oracle import adamw as oa
    from oracle import masks as om
    from oracle import retrain as orc
    from sparseforge_amd import sparse_modeling as sm
    from sparseforge_amd import utils as U
    from sparseforge_amd.retrain import RetrainStep

    dev = cuda_device
    shape, student, teacher, opt, rc = _build(dev)
    teacher_np = {k: v.detach().cpu().numpy() for k, v in teacher.named_parameters()}
    names = orc.sparse_names(shape)
    ocfg = om.full_config(**CFG)
    captured = {}

    def grab(model):
        captured.clear()
        for n, p in model.named_parameters():
            if p.grad is not None:
                captured[n] = p.grad.detach().cpu().numpy().copy()

    step = RetrainStep(student, teacher, opt, rc, on_grads=grab)
    gen = torch.Generator().manual_seed(11)
    for it in (1, 2):
        batches = [(torch.randint(0, shape.vocab_size, (2, 64), generator=gen),
                    torch.randint(0, shape.vocab_size, (2, 64), generator=gen)) for _ in range(2)]
        before = _snapshot(student, opt)
        seed0 = 100 * it
        monkeypatch.setattr(U, "_seed_counter", itertools.count(seed0))
        res = step(it, [(X.to(dev), Y.to(dev)) for X, Y in batches])
        assert not res.skipped
        after = _snapshot(student, opt)
        ref = orc.step(before, teacher_np, shape, ocfg, STEP, it,
                       [(X.numpy(), Y.numpy()) for X, Y in batches], seed0)
        # loss, clipped gradients, Hutchinson accumulator against the float64 chain
        assert abs(res.loss - ref["loss"]) <= 1e-5 * abs(ref["loss"]), (it, res.loss, ref["loss"])
        assert set(captured) == set(ref["grads"]), sorted(set(captured) ^ set(ref["grads"]))
        for k, gref in ref["grads"].items():
            assert rel(captured[k], gref) < 1e-5, (it, k, rel(captured[k], gref))
        for n in names:
            assert rel(after[n + ".hessian_diag"], ref["hessian"][n]) < 1e-5, (it, n)
        # AdamW on the GPU's own inputs: bit for bit
        for k in ref["grads"]:
            mask = before[k[:-7] + ".mask"] if (k.endswith(".weight") and k[:-7] in names) else None
            p1, m1, v1, _ = oa.step(before[k], captured[k], before.get(k + ".exp_avg", np.zeros_like(before[k])),
                                    before.get(k + ".exp_avg_sq", np.zeros_like(before[k])), None, mask,
                                    after[k + ".step"], STEP["lr"], STEP["betas"], STEP["eps"],
                                    STEP["weight_decay"] if before[k].ndim >= 2 else 0.0)
            assert np.array_equal(after[k], p1), (it, k)
            assert np.array_equal(after[k + ".exp_avg"], m1) and np.array_equal(after[k + ".exp_avg_sq"], v1), (it, k)
        # mask update on the GPU's own post-step W and H
        mods = dict(student.named_modules())
        for n in names:
            new, _fr, flips, hx = om.layer_update_mask(ocfg, it, after[n + ".weight"], after[n + ".hessian_diag"],
                                                       before[n + ".mask"], None, None, ref["lambda_mid"])
            got = after[n + ".mask"]
            assert np.abs(got - new).max() <= 1e-6, (it, n, np.abs(got - new).max())
            assert np.array_equal(om.hard_mask_from_soft(got, "nm_2_4"), om.hard_mask_from_soft(new, "nm_2_4"))
            assert int(mods[n].weight.flipped_mask) == flips, (it, n)
            assert after[n + ".hx"] == hx
        # end to end: the oracle's own chain.  Adam's step -lr m / (sqrt(v) + eps) is ill-conditioned where the
        # gradient is near zero (its sign is decided by the last ulps), so such entries may differ by up to two
        # learning-rate steps; entries with a clear gradient agree within 1e-5 of the tensor's scale
        for k, gref in ref["grads"].items():
            d = np.abs(after[k].astype(np.float64) - ref["state"][k])
            clear = np.abs(gref) > 1e-3 * np.abs(gref).max()
            scale = np.abs(ref["state"][k]).max()
            assert d[clear].max(initial=0.0) <= 1e-5 * scale, (it, k, d[clear].max(initial=0.0) / scale)
            assert d.max() <= 2 * STEP["lr"] + 1e-5 * scale, (it, k)
        for n in names:
            dm = np.abs(after[n + ".mask"] - ref["state"][n + ".mask"])
            assert dm.max() <= float(CFG["mask_lr"]) and float((dm > 1e-5).mean()) < 0.01, (it, n, dm.max())
        assert any(isinstance(m, sm.SparseLinear) and m.hardening_x < 1 for m in student.modules())
