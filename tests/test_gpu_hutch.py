"""GPU parity of the Hutchinson kernels (sf_rademacher, sf_rademacher_dot,
sf_hutchinson_update) and of the drop-in update_hessian_hutchinson
(legacy/utils.py:714-869) against the oracle and the reference's outputs.

Bar: the counter-RNG probe and the f32 update are bit-exact against the
oracle; the end-to-end update (double backward through the masked linear)
within 1e-5 relative of the reference's outputs given its own probes.
"""
import itertools

import numpy as np
import pytest
import torch

from conftest import load_golden

pytestmark = pytest.mark.gpu


def test_rademacher_matches_oracle(cuda_device):
    from oracle import hutchinson as oh
    from sparseforge_amd import utils

    for n, seed in ((1, 3), (129, 2 ** 63 + 11), (1_000_003, 424242)):
        v = utils.rademacher((n,), torch.float32, cuda_device, seed).cpu().numpy()
        assert np.array_equal(v, oh.rademacher(seed, n))
        vb = utils.rademacher((n,), torch.bfloat16, cuda_device, seed).float().cpu().numpy()
        assert np.array_equal(vb, oh.rademacher(seed, n))


def test_probe_dot_and_update_bit_exact(cuda_device):
    from oracle import hutchinson as oh
    from sparseforge_amd import utils

    rng = np.random.default_rng(8)
    n = 300_007
    g = rng.standard_normal(n).astype(np.float32)
    hvp = rng.standard_normal(n).astype(np.float32)
    H = (rng.random(n) * 1e-3).astype(np.float32)
    seed = 77
    v = oh.rademacher(seed, n)
    dot = utils._ProbeDot.apply(torch.from_numpy(g).to(cuda_device), seed, None).item()
    assert abs(dot - float(np.dot(g.astype(np.float64), v))) <= 1e-5 * np.abs(g).sum()
    Hd = torch.from_numpy(H.copy()).to(cuda_device)
    utils.hutchinson_update_(Hd, torch.from_numpy(hvp).to(cuda_device), 0.98, seed=seed)
    assert np.array_equal(Hd.cpu().numpy(), oh.update(H, hvp, v, 0.98))
    Hd2 = torch.from_numpy(H.copy()).to(cuda_device)
    utils.hutchinson_update_(Hd2, torch.from_numpy(hvp).to(cuda_device), 0.98, v=torch.from_numpy(v).to(cuda_device))
    assert torch.equal(Hd2, Hd)


def _quadratic_layer(cuda_device, r):
    from sparseforge_amd import sparse_modeling as sm

    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio",
                                beta=0.98)
    layer = sm.SparseLinear(48, 24, sparselinear_config=cfg, bias=False).to(cuda_device)
    with torch.no_grad():
        layer.weight.copy_(torch.from_numpy(r["W"]))
        layer.mask.copy_(torch.from_numpy(r["mask"]))
        layer.hessian_diag.copy_(torch.from_numpy(r["init_H"]))
    return layer


def test_update_hessian_hutchinson_matches_reference(cuda_device):
    from sparseforge_amd import utils

    r = load_golden("hutch_quadratic_f32")
    layer = _quadratic_layer(cuda_device, r)
    model = torch.nn.Sequential(layer)
    x = torch.from_numpy(r["x"]).to(cuda_device)
    y = torch.from_numpy(r["y"]).to(cuda_device)
    for j in range(3):
        loss = 0.5 * ((model(x) - y) ** 2).sum()
        utils.update_hessian_hutchinson(model, loss, probes=[torch.from_numpy(r[f"v{j}"])])
        got, ref = layer.hessian_diag.detach().cpu().numpy(), r[f"H{j}"]
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max(), j
        with torch.no_grad():
            layer.hessian_diag.copy_(torch.from_numpy(ref))


def test_update_hessian_hutchinson_counter_probe(cuda_device, monkeypatch):
    """Default path: the probe is regenerated from the seed; equals the oracle with the same probe."""
    from oracle import hutchinson as oh
    from sparseforge_amd import utils

    r = load_golden("hutch_quadratic_f32")
    layer = _quadratic_layer(cuda_device, r)
    monkeypatch.setattr(utils, "_seed_counter", itertools.count(9001))
    x = torch.from_numpy(r["x"]).to(cuda_device)
    y = torch.from_numpy(r["y"]).to(cuda_device)
    loss = 0.5 * ((layer(x) - y) ** 2).sum()
    utils.update_hessian_hutchinson(torch.nn.Sequential(layer), loss)
    v = oh.rademacher(9001, 24 * 48).reshape(24, 48)
    ref = oh.update(r["init_H"], oh.quadratic_hvp(r["x"], v).astype(np.float32), v, 0.98)
    got = layer.hessian_diag.detach().cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
