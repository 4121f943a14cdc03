"""Pins the distillation KL oracle (oracle/distill.py) -- CPU only.

* the reference's own output on a fixed input (tests/golden/ref_kl_basic_f32.npz,
  written by tests/golden/make_reference_golden.py);
* the closed form F.kl_div(log_softmax(s/T), log_softmax(t/T), log_target=True,
  reduction='sum') * T^2 / tokens (torch, the library the reference calls);
* the chunk skip: a NaN logit drops exactly its chunk of rows;
* the gradient against torch autograd of the closed form.
"""
import numpy as np
import torch
import torch.nn.functional as F

from conftest import load_golden
from oracle import distill as od


def _closed_form(s, t, T):
    s = torch.from_numpy(s).double().clamp(-100, 100) / T
    t = torch.from_numpy(t).double().clamp(-100, 100) / T
    n = s.reshape(-1, s.shape[-1]).shape[0]
    return F.kl_div(F.log_softmax(s, -1), F.log_softmax(t, -1), log_target=True, reduction="sum") * T * T / n


def test_kl_matches_reference_golden():
    r = load_golden("kl_basic_f32")
    got = od.kl_loss(r["s"], r["t"], 2.0)
    np.testing.assert_allclose(got, float(r["kl"]), rtol=2e-6)


def test_kl_matches_closed_form():
    rng = np.random.default_rng(0)
    s = (rng.standard_normal((3, 50, 700)) * 6).astype(np.float32)
    t = (rng.standard_normal((3, 50, 700)) * 6).astype(np.float32)
    s[0, 0, 0], t[1, 2, 3] = 500.0, -300.0
    for T in (1.0, 2.0, 3.5):
        np.testing.assert_allclose(od.kl_loss(s, t, T), float(_closed_form(s, t, T)), rtol=2e-6)
    assert od.kl_loss(s, s, 2.0) == 0.0


def test_kl_nan_skips_its_chunk():
    rng = np.random.default_rng(1)
    v = 64
    s = rng.standard_normal((5000, v)).astype(np.float32)
    t = rng.standard_normal((5000, v)).astype(np.float32)
    assert od.chunk_rows(v) == 2048
    s_nan = s.copy()
    s_nan[3000, 5] = np.nan  # chunk 1 = rows 2048..4095
    keep = np.r_[0:2048, 4096:5000]
    part = _closed_form(s[keep], t[keep], 2.0).item() * len(keep) / 5000
    np.testing.assert_allclose(od.kl_loss(s_nan, t, 2.0), part, rtol=2e-6)
    g = od.kl_grad(s_nan, t, 2.0)
    assert (g[2048:4096] == 0).all() and np.abs(g[:2048]).max() > 0
    assert od.chunk_rows(50001) == 512 and od.chunk_rows(100001) == 128


def test_kl_grad_matches_autograd():
    rng = np.random.default_rng(2)
    s = (rng.standard_normal((40, 300)) * 30).astype(np.float32)  # some logits beyond the clamp
    t = (rng.standard_normal((40, 300)) * 5).astype(np.float32)
    st = torch.from_numpy(s).double().requires_grad_(True)
    loss = F.kl_div(F.log_softmax(st.clamp(-100, 100) / 2.0, -1),
                    F.log_softmax(torch.from_numpy(t).double().clamp(-100, 100) / 2.0, -1),
                    log_target=True, reduction="sum") * 4.0 / 40
    loss.backward()
    np.testing.assert_allclose(od.kl_grad(s, t, 2.0), st.grad.numpy(), rtol=1e-9, atol=1e-12)
    assert (od.kl_grad(s, t, 2.0)[np.abs(s) > 100] == 0).all()


def test_reference_mutates_f32_logits_in_place():
    """Recorded quirk: for float32 logits the reference's .float() is the tensor itself, so its
    clamp_ / mul_(1/T) rewrite the caller's logits (the loss is unaffected).  The device path
    leaves its inputs alone."""
    r = load_golden("kl_basic_f32")
    assert np.array_equal(r["s_after"], (np.clip(r["s"], -100, 100) * np.float32(0.5)).astype(np.float32))
    assert np.array_equal(r["t_after"], (np.clip(r["t"], -100, 100) * np.float32(0.5)).astype(np.float32))
