"""Pins the float64 step restatement (oracle/retrain.py) on the CPU.

* its KL equals oracle.distill.kl_loss (pinned against the reference's own
  output) on logits with clamped entries, and its gradient equals
  oracle.distill.kl_grad;
* its straight-through linear gives oracle.linear.backward's gradients and,
  for a quadratic loss, oracle.hutchinson.quadratic_hvp as the double-backward
  Hessian-vector product (the mask drops out);
* with all-one masks and no SLoRB the student forward equals the dense
  teacher forward of the same weights;
* a dropped Hutchinson probe term or mask update is visible: the step changes
  hessian_diag and the soft masks, and the flip counts are reported.
"""
import numpy as np
import torch

from oracle import distill as od
from oracle import hutchinson as oh
from oracle import linear as ol
from oracle import retrain as orc


def test_kl_restatement_matches_pinned_oracle():
    rng = np.random.default_rng(5)
    s = (rng.standard_normal((2, 37, 300)) * 4).astype(np.float32)
    t = (rng.standard_normal((2, 37, 300)) * 4).astype(np.float32)
    s[0, 3, 7] = 250.0
    t[1, 5, 9] = -400.0
    st = torch.tensor(s, dtype=torch.float64, requires_grad=True)
    kl = orc.kl_loss(st, torch.tensor(t, dtype=torch.float64))
    assert abs(float(kl.detach()) - float(od.kl_loss(s, t))) <= 1e-6 * abs(float(kl.detach()))
    (g,) = torch.autograd.grad(kl, st)
    ref = od.kl_grad(s.reshape(-1, 300), t.reshape(-1, 300)).reshape(g.shape)
    assert np.abs(g.numpy() - ref).max() <= 1e-6 * np.abs(ref).max()


def test_ste_linear_gradients_and_hvp():
    rng = np.random.default_rng(6)
    T, IN, OUT = 40, 24, 16
    x = rng.standard_normal((T, IN))
    W = rng.standard_normal((OUT, IN)) * 0.1
    E = rng.random((OUT, IN))
    gy = rng.standard_normal((T, OUT))
    xt = torch.tensor(x, requires_grad=True)
    Wt = torch.tensor(W, requires_grad=True)
    y = orc._STE.apply(xt, Wt, torch.tensor(E))
    y.backward(torch.tensor(gy))
    ref = ol.backward(x, W, E, gy, False, dtype=np.float64)
    np.testing.assert_allclose(xt.grad.numpy(), ref["dx"], rtol=1e-12)
    np.testing.assert_allclose(Wt.grad.numpy(), ref["dW"], rtol=1e-12)
    tgt = torch.tensor(rng.standard_normal((T, OUT)))
    v = torch.tensor(oh.rademacher(9, OUT * IN).reshape(OUT, IN), dtype=torch.float64)
    W2 = torch.tensor(W, requires_grad=True)
    loss = 0.5 * ((orc._STE.apply(torch.tensor(x), W2, torch.tensor(E)) - tgt) ** 2).sum()
    (g,) = torch.autograd.grad(loss, W2, create_graph=True)
    (hvp,) = torch.autograd.grad((g * v).sum(), W2)
    np.testing.assert_allclose(hvp.numpy(), oh.quadratic_hvp(x, v.numpy()), rtol=1e-10, atol=1e-12)


def _tiny_state(seed=0):
    from sparseforge_amd.llama import LlamaShape

    shape = LlamaShape(vocab_size=64, hidden_size=32, intermediate_size=64, num_hidden_layers=1,
                       num_attention_heads=2)
    rng = np.random.default_rng(seed)
    h, f, V = shape.hidden_size, shape.intermediate_size, shape.vocab_size
    P = {"embed_tokens.weight": rng.standard_normal((V, h)) * 0.02, "norm.weight": np.ones(h),
         "lm_head.weight": rng.standard_normal((V, h)) * 0.02,
         "layers.0.input_layernorm.weight": np.ones(h), "layers.0.post_attention_layernorm.weight": np.ones(h)}
    dims = {"self_attn.q_proj": (h, h), "self_attn.k_proj": (h, h), "self_attn.v_proj": (h, h),
            "self_attn.o_proj": (h, h), "mlp.gate_proj": (f, h), "mlp.up_proj": (f, h), "mlp.down_proj": (h, f)}
    for n, shp in dims.items():
        P[f"layers.0.{n}.weight"] = rng.standard_normal(shp) * 0.02
    return shape, {k: v.astype(np.float32) for k, v in P.items()}, rng


def test_student_with_unit_masks_equals_dense_teacher():
    shape, P, rng = _tiny_state()
    Pt = {k: torch.tensor(v, dtype=torch.float64) for k, v in P.items()}
    E = {n: torch.ones_like(Pt[n + ".weight"]) for n in orc.sparse_names(shape)}
    idx = torch.tensor(rng.integers(0, shape.vocab_size, (2, 9)))
    a = orc.forward(Pt, E, shape, idx, True, False)
    b = orc.forward(Pt, None, shape, idx, False, False)
    np.testing.assert_allclose(a.detach().numpy(), b.numpy(), rtol=1e-12, atol=1e-14)
    # the causal mask: the first position's logits do not depend on later tokens
    idx2 = idx.clone()
    idx2[:, 1:] = (idx2[:, 1:] + 1) % shape.vocab_size
    c = orc.forward(Pt, None, shape, idx2, False, False)
    np.testing.assert_allclose(c[:, 0].numpy(), b[:, 0].numpy(), rtol=1e-12)
    assert np.abs(c[:, 1:].numpy() - b[:, 1:].numpy()).max() > 1e-6


def test_step_updates_hessian_masks_and_parameters():
    from oracle import masks as om

    shape, P, rng = _tiny_state(1)
    state = dict(P)
    for n in orc.sparse_names(shape):
        W = P[n + ".weight"]
        state[n + ".mask"] = rng.random(W.shape).astype(np.float32)
        state[n + ".hessian_diag"] = (rng.random(W.shape) * 1e-3 + 1e-6).astype(np.float32)
        state[n + ".hx"] = 0.75
    teacher = {k: v for k, v in P.items()}
    cfg = om.full_config(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio", beta=0.98,
                         mask_update_period=1, sparsity_warmup_steps=0, mask_hardening_start=0,
                         mask_hardening_duration=4, mask_penalty_mode="nm_2_4", mask_penalty_lr=0.1)
    step_cfg = dict(grad_accum=2, hardness_task=1.0, hardness_kldiv=1.0, lambda_mid_max=0.1, sparsity_ratio=0.5,
                    sparsity_alpha=0.2, grad_clip=1.0, hutchinson=True, mask_penalty_mode="nm_2_4", lr=1e-3,
                    decay=0.0, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    batches = [(rng.integers(0, 64, (2, 8)), rng.integers(0, 64, (2, 8))) for _ in range(2)]
    out = orc.step(state, teacher, shape, cfg, step_cfg, 1, batches, 7)
    new = out["state"]
    for n in orc.sparse_names(shape):
        assert not np.array_equal(new[n + ".hessian_diag"], state[n + ".hessian_diag"])
        assert not np.array_equal(new[n + ".mask"], state[n + ".mask"])
        assert new[n + ".hx"] == 0.75  # hardening at step 1 of a 4-step window starting at 0
        # hessian_diag moved by (1 - beta) clamp(hvp v, 0) exactly as hutchinson.update says
        v = oh.rademacher(7 + orc.sparse_names(shape).index(n), state[n + ".mask"].size).reshape(
            state[n + ".mask"].shape)
        np.testing.assert_array_equal(new[n + ".hessian_diag"],
                                      oh.update(state[n + ".hessian_diag"], out[n + ".hvp"].astype(np.float32), v,
                                                0.98))
    assert out["grad_norm"] > 0 and set(out["flips"]) == set(orc.sparse_names(shape))
