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


def test_oracle_matches_reference_ste_decay_golden():
    """FusedMaskedLinearSTE.apply with decay != 0 and scale != 1 (the reference's own outputs): the
    forward carries the scale, dx does not, dW carries decay * W * [mask < 0.5] (mask exactly 0.5
    is kept), and the Hessian-vector product by double backward adds decay * v * [mask < 0.5]."""
    from oracle import hutchinson as oh

    r = load_golden("ste_decay_f32")
    W, b, M = r["W"], r["b"], r["mask"]
    x = r["x"].reshape(-1, W.shape[1])
    gy = r["gy"].reshape(-1, W.shape[0])
    decay, scale = float(r["decay"]), float(r["scale"])
    y = ol.forward(x, W, M, b, scale)
    assert rel(y, r["y"].reshape(y.shape)) < 1e-5
    g = ol.backward(x, W, M, gy, True, decay=decay)
    assert rel(g["dx"], r["dx"].reshape(g["dx"].shape)) < 1e-5
    assert rel(g["dW"], r["dW"]) < 1e-5
    assert rel(g["db"], r["db"]) < 1e-5
    # the decay term itself (about 1e-4 of dW's scale, so a relative bar on dW cannot see it): the
    # reference's dW minus the straight-through product is decay * W * [mask < 0.5], zero at mask == 0.5
    x64, gy64 = x.astype(np.float64), gy.astype(np.float64)
    term = decay * W.astype(np.float64) * (M < 0.5)
    resid = r["dW"].astype(np.float64) - gy64.T @ x64
    tol = 1e-6 * np.abs(r["dW"]).max()
    assert np.abs(resid - term).max() < tol
    assert np.abs(term).max() > 100 * tol and np.all(term[M == 0.5] == 0) and np.any(M == 0.5)
    # the reference's HVP is two chained f32 products (x^T x then along v): f32 rounding of both
    hvp = oh.quadratic_hvp(x, r["v"], M, decay)
    assert rel(hvp, r["hvp"]) < 3e-5
    h_resid = r["hvp"].astype(np.float64) - oh.quadratic_hvp(x, r["v"])
    h_tol = 2e-5 * np.abs(r["hvp"]).max()  # f32 rounding of the reference's HVP (~350) over 80 + 64 terms
    assert np.abs(h_resid - decay * r["v"] * (M < 0.5)).max() < h_tol < decay / 5
