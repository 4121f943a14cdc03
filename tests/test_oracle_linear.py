"""Pins the masked-linear oracle (oracle/linear.py) on the CPU.

* against the reference's own FusedMaskedLinearSTE + SLoRB outputs and
  gradients (tests/golden/ref_linear_slorb_f32.npz) at hx = 1, 0.4, 0;
* against torch.autograd on the dense equivalent, which fixes every
  transpose of dx / dP / dS (the STE parts are checked as closed forms).
"""
import numpy as np
import torch

from conftest import load_golden
from oracle import linear as ol


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def test_oracle_matches_reference_golden():
    r = load_golden("linear_slorb_f32")
    W, b, M, P, S = r["W"], r["bias"], r["mask"], r["P"], r["S"]
    for j in range(3):
        hx = float(r[f"hx{j}"])
        x = r[f"x{j}"].reshape(-1, W.shape[1])
        gy = r[f"gy{j}"].reshape(-1, W.shape[0])
        E = ol.effective_mask(M, hx, "nm_2_4")
        s = ol.weight_scale(hx, 2.0) if hx < 1.0 - 1e-6 else 1.0
        y = ol.forward(x, W, E, b, s, P, S)
        assert rel(y, r[f"y{j}"].reshape(y.shape)) < 1e-5, j
        g = ol.backward(x, W, E, gy, True, P, S)
        assert rel(g["dx"], r[f"dx{j}"].reshape(g["dx"].shape)) < 1e-5, j
        for k in ("dW", "db", "dP", "dS"):
            assert rel(g[k], r[f"{k}{j}"]) < 1e-5, (j, k)


def test_oracle_matches_autograd_of_dense_equivalent():
    rng = np.random.default_rng(3)
    T, IN, OUT, R = 33, 24, 16, 4
    x = rng.standard_normal((T, IN))
    W = rng.standard_normal((OUT, IN))
    E = rng.random((OUT, IN))
    P = rng.standard_normal((R, IN))
    S = rng.standard_normal((OUT, R))
    b = rng.standard_normal(OUT)
    gy = rng.standard_normal((T, OUT))
    xt = torch.tensor(x, requires_grad=True)
    Pt = torch.tensor(P, requires_grad=True)
    St = torch.tensor(S, requires_grad=True)
    Wt = torch.tensor(W, requires_grad=True)
    bt = torch.tensor(b, requires_grad=True)
    y = xt @ (Wt * torch.tensor(E)).t() + bt + (xt @ Pt.t()) @ St.t()
    y.backward(torch.tensor(gy))
    np.testing.assert_allclose(ol.forward(x, W, E, b, 1.0, P, S, np.float64), y.detach().numpy(), rtol=1e-12)
    g = ol.backward(x, W, E, gy, True, P, S, dtype=np.float64)
    np.testing.assert_allclose(g["dx"], xt.grad.numpy(), rtol=1e-12)
    np.testing.assert_allclose(g["dP"], Pt.grad.numpy(), rtol=1e-12)
    np.testing.assert_allclose(g["dS"], St.grad.numpy(), rtol=1e-12)
    np.testing.assert_allclose(g["db"], bt.grad.numpy(), rtol=1e-12)
    # straight-through: dW is the gradient w.r.t. the masked product, not masked again
    np.testing.assert_allclose(g["dW"], Wt.grad.numpy() / E, rtol=1e-9)
    # SR-STE decay adds decay * W where E < 0.5
    g2 = ol.backward(x, W, E, gy, True, decay=0.25, dtype=np.float64)
    np.testing.assert_allclose(g2["dW"] - g["dW"], 0.25 * W * (E < 0.5), atol=1e-12)


def test_weight_scale_and_flops():
    assert ol.weight_scale(0.0, 2.0) == 2.0 and ol.weight_scale(1.0, 2.0) == 1.0
    assert ol.flops_fwd_bwd(8192, 4096, 4096) == 6 * 8192 * 4096 * 4096
