"""Pins the Hutchinson oracle (oracle/hutchinson.py) on the CPU.

* SplitMix64 against the published first outputs of the stream seeded with
  1234567 (the generator's reference test vector).
* The update against the reference's own outputs
  (tests/golden/ref_hutch_quadratic_f32.npz: update_hessian_hutchinson on a
  quadratic loss with the reference's probes), with the HVP in closed form.
* The closed-form HVP against torch.autograd double backward of the same
  loss through a straight-through masked product.
* Estimator properties: E[est] = diag(x^T x) in every row (Monte Carlo), and
  est is the exact diagonal for any probe when x^T x is diagonal.
"""
import numpy as np
import torch

from conftest import load_golden
from oracle import hutchinson as oh


def test_splitmix64_published_vector():
    got = oh.splitmix64(1234567, np.arange(5))
    assert [int(x) for x in got] == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                                     4593380528125082431, 16408922859458223821]


def test_rademacher_bits_and_balance():
    v = oh.rademacher(99, 1 << 16)
    assert set(np.unique(v)) == {-1.0, 1.0}
    assert abs(float(v.mean())) < 0.02
    h = int(oh.splitmix64(99, np.array([0]))[0])
    assert [1.0 if (h >> i) & 1 else -1.0 for i in range(64)] == list(v[:64])


def test_update_matches_reference_golden():
    r = load_golden("hutch_quadratic_f32")
    H = r["init_H"]
    for j in range(3):
        hvp = oh.quadratic_hvp(r["x"], r[f"v{j}"]).astype(np.float32)
        H = oh.update(H, hvp, r[f"v{j}"], 0.98)
        np.testing.assert_allclose(H, r[f"H{j}"], rtol=2e-5, atol=1e-9)
        H = r[f"H{j}"]


def test_closed_form_hvp_matches_autograd_double_backward():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((40, 12))
    y = rng.standard_normal((40, 9))
    W = rng.standard_normal((9, 12))
    M = rng.random((9, 12))
    v = np.where(rng.random((9, 12)) < 0.5, -1.0, 1.0)

    class STE(torch.autograd.Function):
        @staticmethod
        def forward(ctx, w, m):
            ctx.save_for_backward(m)
            return w * m

        @staticmethod
        def backward(ctx, g):  # straight-through: the mask does not scale the weight gradient
            return g, None

    Wt = torch.tensor(W, requires_grad=True)
    # the reference's STE backward: dW = gy^T x with gy from the masked forward
    out = torch.tensor(x) @ STE.apply(Wt, torch.tensor(M)).t()
    loss = 0.5 * ((out - torch.tensor(y)) ** 2).sum()
    (g,) = torch.autograd.grad(loss, [Wt], create_graph=True)
    (hvp,) = torch.autograd.grad((g * torch.tensor(v)).sum(), [Wt])
    np.testing.assert_allclose(hvp.numpy(), oh.quadratic_hvp(x, v), rtol=1e-10)


def test_estimator_mean_and_diagonal_case():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((30, 8))
    acc = np.zeros((5, 8))
    n = 4000
    for s in range(n):
        v = oh.rademacher(1000 + s, 40).reshape(5, 8).astype(np.float64)
        acc += oh.quadratic_hvp(x, v) * v
    diag = np.broadcast_to(np.diag(x.T @ x)[None, :], acc.shape)
    np.testing.assert_allclose(acc / n, diag, rtol=0.15, atol=0.6)
    # diagonal x^T x: est equals the diagonal exactly for any probe
    xd = np.diag(np.arange(1.0, 9.0))
    v = oh.rademacher(7, 40).reshape(5, 8).astype(np.float64)
    np.testing.assert_allclose(oh.quadratic_hvp(xd, v) * v, np.broadcast_to(np.diag(xd.T @ xd), (5, 8)), rtol=1e-12)
