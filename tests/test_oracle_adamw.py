"""Pins the AdamW oracle (oracle/adamw.py) on the CPU.

* torch.optim.AdamW(foreach=False) has the same decoupled-decay update; with
  decay = 0 and l1 = 0 the two must agree, and with decay != 0 the oracle
  equals torch's AdamW run on the gradient with the masked-decay term added.
* The reference's own outputs (tests/golden/ref_adamw_*.npz, AdamW.step of
  legacy/adamw.py) within the fp32 bar of 1e-6.
* The per-op rounding the oracle assumes for torch's CPU kernels.
* The L1 term in closed form.
"""
import ast

import numpy as np
import pytest
import torch

from conftest import load_golden
from oracle import adamw as oa


def _torch_adamw(w0, grads, lr, betas, eps, wd, amsgrad):
    p = torch.nn.Parameter(torch.tensor(w0))
    opt = torch.optim.AdamW([p], lr=lr, betas=betas, eps=eps, weight_decay=wd, amsgrad=amsgrad, foreach=False)
    out = []
    for g in grads:
        p.grad = torch.tensor(g)
        opt.step()
        st = opt.state[p]
        out.append((p.detach().numpy().copy(), st["exp_avg"].numpy().copy(), st["exp_avg_sq"].numpy().copy()))
    return out


@pytest.mark.parametrize("amsgrad", [False, True])
def test_matches_torch_adamw_without_mask_terms(amsgrad):
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((33, 17)) * 0.05).astype(np.float32)
    grads = [(rng.standard_normal(w.shape) * 1e-2).astype(np.float32) for _ in range(5)]
    ref = _torch_adamw(w, grads, 2e-3, (0.9, 0.95), 1e-8, 0.1, amsgrad)
    p, m, v, x = w, np.zeros_like(w), np.zeros_like(w), np.zeros_like(w)
    for k, g in enumerate(grads):
        p, m, v, x = oa.step(p, g, m, v, x, None, k + 1, 2e-3, (0.9, 0.95), 1e-8, 0.1, amsgrad=amsgrad)
        np.testing.assert_allclose(p, ref[k][0], rtol=0, atol=1e-7)
        np.testing.assert_allclose(m, ref[k][1], rtol=0, atol=1e-9)
        np.testing.assert_allclose(v, ref[k][2], rtol=1e-6, atol=0)


def test_masked_decay_is_a_gradient_term():
    """decay != 0 equals torch's AdamW on g + decay * p_decayed * (1 - mask)."""
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((16, 24)) * 0.05).astype(np.float32)
    mask = rng.random(w.shape).astype(np.float32)
    g = (rng.standard_normal(w.shape) * 1e-2).astype(np.float32)
    lr, wd, dec = 1e-2, 0.05, 3e-3
    p_dec = (w * np.float32(1 - lr * wd)).astype(np.float32)
    g_eff = (g.astype(np.float64) + dec * (p_dec * (1 - mask)).astype(np.float32)).astype(np.float32)
    ref = _torch_adamw(w, [g_eff], lr, (0.9, 0.999), 1e-8, wd, False)[0]
    p, m, v, _ = oa.step(w, g, np.zeros_like(w), np.zeros_like(w), None, mask, 1, lr, (0.9, 0.999), 1e-8, wd,
                         decay=dec)
    np.testing.assert_allclose(p, ref[0], rtol=0, atol=1e-7)
    np.testing.assert_allclose(m, ref[1], rtol=1e-6, atol=0)


@pytest.mark.parametrize("name", ["adamw_plain", "adamw_decay_l1", "adamw_amsgrad"])
def test_matches_reference_golden(name):
    r = load_golden(name)
    h = ast.literal_eval(str(r["cfg"]))
    n = sum(1 for k in r if k.startswith("decay"))
    w, b = r["init_w"], r["init_b"]
    sw = [np.zeros_like(w) for _ in range(3)]
    sb = [np.zeros_like(b) for _ in range(3)]
    for j in range(n):
        d = float(r[f"decay{j}"])
        kw = dict(lr=h["lr"], betas=h["betas"], eps=h["eps"], weight_decay=h["weight_decay"], decay=d,
                  l1=h["adaptive_l1_decay"], amsgrad=h["amsgrad"])
        w, sw[0], sw[1], sw[2] = oa.step(w, r[f"gw{j}"], sw[0], sw[1], sw[2], r["mask"], j + 1, **kw)
        b, sb[0], sb[1], sb[2] = oa.step(b, r[f"gb{j}"], sb[0], sb[1], sb[2], None, j + 1, **kw)
        for got, key in ((w, "w"), (b, "b"), (sw[0], "m"), (sw[1], "v")):
            np.testing.assert_allclose(got, r[f"{key}{j}"], rtol=0, atol=1e-6, err_msg=f"{name} {key}{j}")
        if h["amsgrad"]:
            np.testing.assert_allclose(sw[2], r[f"vmax{j}"], rtol=0, atol=1e-6)


def test_torch_cpu_op_rounding_assumed_by_the_oracle():
    g = torch.Generator().manual_seed(2)
    w, y, z = (torch.rand(50000, generator=g) for _ in range(3))
    z = z + 0.5
    W, Y, Z = w.numpy(), y.numpy(), z.numpy()
    f32, f64 = np.float32, np.float64
    assert np.array_equal(torch.add(w, y, alpha=0.37).numpy(), (Y.astype(f64) * f32(0.37) + W).astype(f32))
    assert np.array_equal(w.clone().addcmul_(y, z, value=0.37).numpy(),
                          ((f32(0.37) * Y).astype(f32).astype(f64) * Z + W).astype(f32))
    assert np.array_equal(w.clone().addcdiv_(y, z, value=-0.37).numpy(),
                          (W + ((f32(-0.37) * Y).astype(f32) / Z).astype(f32)).astype(f32))
    assert np.array_equal((w / 1.2345678).numpy(), (W / f32(1.2345678)).astype(f32))


def test_l1_term_closed_form():
    """With lr * wd = 0, zero gradient history and a mask, the L1 step is -lr * l1 * sign(p) / (sqrt(v) + eps)."""
    w = np.array([[0.3, -0.2], [0.0, 0.1]], np.float32)
    g = np.zeros_like(w)
    p, m, v, _ = oa.step(w, g, np.zeros_like(w), np.zeros_like(w), None, np.ones_like(w), 1, 0.1, (0.9, 0.999), 1e-3,
                         0.0, decay=0.0, l1=0.5)
    np.testing.assert_allclose(p, w - 0.1 * 0.5 * np.sign(w) / 1e-3, rtol=1e-6)


def test_bytes_per_param_of_the_7b_arena():
    assert oa.bytes_per_param() == 32
