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


@pytest.mark.parametrize("n", [300_007, 300_008, 4096 * 1027])
def test_probe_dot_and_update_bit_exact(cuda_device, n):
    """n % 4 == 0 takes the vectorised update (one hash per 4 elements), the others the scalar one."""
    from oracle import hutchinson as oh
    from sparseforge_amd import utils

    rng = np.random.default_rng(8)
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


@pytest.mark.parametrize("autocast,tol", [(False, 1e-5), (True, 2e-2)])
def test_hvp_with_slorb_and_mixed_mask(cuda_device, autocast, tol):
    """Hessian-vector product of 1/2 ||y - t||^2 through a SparseLinear with SLoRB (rank 32) and a mixed
    hardening mask (hardening_x = 0.5), taken jointly over (W, P, S) so every second-order branch of the
    backward runs (the SLoRB terms of d/d gy, d/dx, d/dW, d/dP, d/dS), against the float64 double backward
    of the straight-through restatement (oracle/retrain._STE plus the SLoRB pair).  With autocast the
    operands are rounded to bf16 first, as autocast does; bar 2e-2 (bf16) / 1e-5 (f32) of each tensor's
    largest magnitude."""
    from oracle import linear as ol
    from oracle import retrain as orc
    from sparseforge_amd import sparse_modeling as sm

    T, IN, OUT, K = 512, 256, 192, 8
    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio",
                                SLoRB=True, SLoRB_k=K, SLoRB_init_type="sum", trainable_projection=True)
    layer = sm.SparseLinear(IN, OUT, sparselinear_config=cfg, bias=False).to(cuda_device)
    g = torch.Generator().manual_seed(31)
    W = torch.randn(OUT, IN, generator=g) * 0.05
    M = torch.rand(OUT, IN, generator=g)
    S = torch.randn(OUT, IN // K, generator=g) * 0.05
    with torch.no_grad():
        layer.weight.copy_(W)
        layer.mask.copy_(M)
        layer.init_SLoRB()
        layer.SLoRB_Weight.copy_(S)
        layer.x_proj.add_(torch.randn(layer.x_proj.shape, generator=g).to(cuda_device) * 0.05)
    layer.hardening_x = 0.5
    P = layer.x_proj.detach().cpu()
    x = torch.randn(T, IN, generator=g)
    t = torch.randn(T, OUT, generator=g)
    params = [layer.weight, layer.x_proj, layer.SLoRB_Weight]
    vs = [torch.randint(0, 2, p.shape, generator=g).float() * 2 - 1 for p in params]
    ctx = torch.autocast("cuda", dtype=torch.bfloat16) if autocast else torch.autocast("cuda", enabled=False)
    with ctx:
        y = layer(x.to(cuda_device))
    loss = 0.5 * ((y.float() - t.to(cuda_device)) ** 2).sum()
    grads = torch.autograd.grad(loss, params, create_graph=True)
    dot = sum((gr.float() * v.to(cuda_device)).sum() for gr, v in zip(grads, vs))
    hvps = torch.autograd.grad(dot, params)
    rb = (lambda a: a.to(torch.bfloat16).double()) if autocast else (lambda a: a.double())  # noqa: E731
    E = torch.tensor(ol.effective_mask(M.numpy(), 0.5, "nm_2_4"))
    Wd, Pd, Sd = (rb(a).requires_grad_(True) for a in (W, P, S))
    xd = rb(x)
    y64 = orc._STE.apply(xd, Wd, rb(E)) + (xd @ Pd.t()) @ Sd.t()
    if autocast:
        y64 = y64.to(torch.bfloat16).double()  # the bf16 output autocast produces
    l64 = 0.5 * ((y64 - t.double()) ** 2).sum()
    g64 = torch.autograd.grad(l64, (Wd, Pd, Sd), create_graph=True)
    h64 = torch.autograd.grad(sum((a * v.double()).sum() for a, v in zip(g64, vs)), (Wd, Pd, Sd))
    for name, got, ref in zip(("W", "P", "S"), hvps, h64):
        err = float((got.double().cpu() - ref).abs().max() / ref.abs().max())
        assert err < tol, (name, err)


@pytest.mark.parametrize("hdt,vdt", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16),
                                     (torch.bfloat16, torch.float32)])
def test_vector_update_equals_scalar_update(cuda_device, hdt, vdt):
    """The vectorised update (probe regenerated, n % 4 == 0) equals the scalar one fed the materialised
    probe, bit for bit, for bf16 accumulators and bf16 Hessian-vector products."""
    from sparseforge_amd import utils

    n = 4096 * 515
    g = torch.Generator(device=cuda_device).manual_seed(4)
    H = (torch.rand(n, generator=g, device=cuda_device) * 1e-3).to(hdt)
    hvp = torch.randn(n, generator=g, device=cuda_device).to(vdt)
    seed = 12345
    a, b = H.clone(), H.clone()
    utils.hutchinson_update_(a, hvp, 0.98, seed=seed)
    v = utils.rademacher((n,), hvp.dtype, cuda_device, seed)
    utils.hutchinson_update_(b, hvp, 0.98, v=v)
    assert torch.equal(a, b)


@pytest.mark.parametrize("hdt,vdt", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.bfloat16),
                                     (torch.float32, torch.float32)])
def test_multi_tensor_update_equals_single_updates(cuda_device, hdt, vdt):
    """hutchinson_update_multi_ (sf_hutchinson_update_multi, 48 tensors per launch) equals one
    hutchinson_update_ per tensor bit for bit: 53 tensors (two launches) of mixed sizes, one not a
    multiple of 4 (it takes the single call), different seeds and betas."""
    from sparseforge_amd import utils

    g = torch.Generator(device=cuda_device).manual_seed(8)
    sizes = [4096 * (1 + (k * 37) % 300) for k in range(52)] + [4099]
    items_a, items_b = [], []
    for k, n in enumerate(sizes):
        H = (torch.rand(n, generator=g, device=cuda_device) * 1e-3).to(hdt)
        hvp = torch.randn(n, generator=g, device=cuda_device).to(vdt)
        beta = 0.98 if k % 3 else 0.9
        items_a.append((H.clone(), hvp, beta, 1000 + k))
        items_b.append((H.clone(), hvp, beta, 1000 + k))
    utils.hutchinson_update_multi_(items_a)
    for H, hvp, beta, seed in items_b:
        utils.hutchinson_update_(H, hvp, beta, seed=seed)
    for (a, *_), (b, *_) in zip(items_a, items_b):
        assert torch.equal(a, b)
