"""GPU parity of the GLU gate/up joint mask update (sf_joint_scores + sf_glu_update_masks).

Bar: masks within 1e-6 (f32) / one bf16 ulp at 1.0 (bf16) of the reference's
own output (tests/golden/ref_glu_joint_f32.npz) and of oracle/masks.py
glu_joint_update; flip counts exact; hardening_x equal.
"""
import ast

import numpy as np
import pytest
import torch

from conftest import load_golden
from oracle import masks as om
from oracle.numerics import BF16, F32

pytestmark = pytest.mark.gpu


def _sm():
    from sparseforge_amd import sparse_modeling as sm

    return sm


def _pair(cfg_kw, Wg, Hg, Mg, Wu, Hu, Mu, tdt, dev, frozen=None):
    sm = _sm()
    mods = []
    for W, H, M in ((Wg, Hg, Mg), (Wu, Hu, Mu)):
        cfg = sm.SparseLinearConfig(**cfg_kw)
        if cfg_kw.get("mask_metric", "") in ("hessian_ratio", "hessian_obd", "hessian"):
            cfg.enable_hutchinson = True
        layer = sm.SparseLinear(W.shape[1], W.shape[0], sparselinear_config=cfg, bias=False).to(tdt).to(dev)
        with torch.no_grad():
            layer.weight.copy_(torch.as_tensor(W).to(tdt))
            layer.hessian_diag.copy_(torch.as_tensor(H).to(tdt))
            layer.mask.copy_(torch.as_tensor(M).to(tdt))
        layer.weight.mask = layer.mask
        mods.append(layer)
    if frozen is not None:
        with torch.no_grad():
            mods[0].frozen_mask_flags.copy_(torch.as_tensor(frozen).to(tdt))
    return mods


def test_glu_joint_matches_reference(cuda_device):
    from sparseforge_amd.glu import glu_joint_update

    r = load_golden("glu_joint_f32")
    kw = ast.literal_eval(str(r["cfg"]))
    gate, up = _pair(kw, r["Wg"], r["Hg"], r["init_Mg"], r["Wu"], r["Hu"], r["init_Mu"], torch.float32, cuda_device)
    for j, step in enumerate((1, 2, 3)):
        idx = torch.from_numpy(r[f"idx{j}"]).to(cuda_device)
        glu_joint_update(gate, up, step, 0.05, sample_idx=idx)
        np.testing.assert_allclose(gate.mask.cpu().numpy(), r[f"Mg{j}"], rtol=0, atol=1e-6)
        np.testing.assert_allclose(up.mask.cpu().numpy(), r[f"Mu{j}"], rtol=0, atol=1e-6)
        assert int(gate.weight.flipped_mask) == int(r[f"flips_g{j}"])
        assert int(up.weight.flipped_mask) == int(r[f"flips_u{j}"])
        assert gate.hardening_x == up.hardening_x == float(r[f"hx{j}"])
        with torch.no_grad():  # continue from the reference state
            gate.mask.copy_(torch.from_numpy(r[f"Mg{j}"]))
            up.mask.copy_(torch.from_numpy(r[f"Mu{j}"]))


CASES = {
    "topn_bin_frozen": dict(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio",
                            mask_penalty_mode="structured_topn", mask_binarize_decay=0.05, freeze_low=0.02,
                            tau_sample_size=4096),
    "structured_beta": dict(mask_type="structured", mask_metric="hessian_obd", mask_penalty_mode="mid",
                            beta_structural_start=0, beta_structural_end=20, temp_init=0.5),
    "nm24_mode_exact": dict(mask_type="structured", structured_exact=True, mask_metric="hessian",
                            mask_penalty_mode="nm_2_4"),
}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", sorted(CASES))
def test_glu_joint_matches_oracle(cuda_device, dtype, case):
    from sparseforge_amd.glu import glu_joint_update

    kw = dict(sparsity_warmup_steps=0, mask_update_period=1, mask_lr=0.1, mask_penalty_lr=0.2, **CASES[case])
    rows, cols = 256, 1024
    g = torch.Generator().manual_seed(len(case))
    Wg, Wu = [(torch.randn(rows, cols, generator=g) * 0.02).to(dtype) for _ in range(2)]
    Hg, Hu = [(torch.rand(rows, cols, generator=g) * 1e-3).to(dtype) for _ in range(2)]
    Mg, Mu = [torch.rand(rows, cols, generator=g).to(dtype) for _ in range(2)]
    frozen = (torch.rand(rows, cols, generator=g) < 0.1).to(dtype) if kw.get("freeze_low", 0) > 0 else None
    gate, up = _pair(kw, Wg, Hg, Mg, Wu, Hu, Mu, dtype, cuda_device, frozen)
    idx = torch.randint(0, rows * cols, (4096,), generator=g)
    step = 7
    glu_joint_update(gate, up, step, 0.05, sample_idx=idx.to(cuda_device))
    odt = F32 if dtype == torch.float32 else BF16
    c = om.full_config(**kw)
    f = lambda t: t.float().numpy()
    ng, nu, fg, fu, hx = om.glu_joint_update(c, step, f(Wg), f(Hg), f(Mg), f(Wu), f(Hu), f(Mu),
                                             None if frozen is None else f(frozen), idx.numpy(), 0.05, odt, odt, odt)
    tol = 1e-6 if odt == F32 else 2 ** -8
    np.testing.assert_allclose(gate.mask.float().cpu().numpy(), ng, rtol=0, atol=tol)
    np.testing.assert_allclose(up.mask.float().cpu().numpy(), nu, rtol=0, atol=tol)
    if odt == F32:
        assert (int(gate.weight.flipped_mask), int(up.weight.flipped_mask)) == (fg, fu)
    assert gate.hardening_x == hx
    if frozen is not None:  # the joint path never writes the frozen flags
        assert torch.equal(gate.frozen_mask_flags.cpu(), frozen)


def test_calculate_model_mask_routes_glu_pairs(cuda_device):
    """calculate_model_mask sends `*.mlp.gate_proj` / `up_proj` through the joint update, the rest per layer."""
    sm = _sm()
    from sparseforge_amd import utils as U

    kw = dict(mask_type="structured", mask_metric="hessian_obd", sparsity_warmup_steps=0, mask_update_period=1,
              mask_lr=0.1, glu_joint_mask=True)

    def lin(i, o):
        cfg = sm.SparseLinearConfig(**kw)
        cfg.enable_hutchinson = True
        return sm.SparseLinear(i, o, sparselinear_config=cfg, bias=False)

    class MLP(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_proj, self.up_proj, self.down_proj = lin(64, 128), lin(64, 128), lin(128, 64)

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.mlp = MLP()

    class Model(torch.nn.Module):  # module names layers.0.mlp.gate_proj etc. (the pair pattern needs the prefix)
        def __init__(self):
            super().__init__()
            self.layers = torch.nn.ModuleList([Block()])

    model = Model().to(cuda_device)
    g = torch.Generator().manual_seed(9)
    with torch.no_grad():
        for m in (model.layers[0].mlp.gate_proj, model.layers[0].mlp.up_proj, model.layers[0].mlp.down_proj):
            m.weight.copy_(torch.randn(m.weight.shape, generator=g) * 0.02)
            m.hessian_diag.copy_(torch.rand(m.weight.shape, generator=g) * 1e-3)
            m.mask.copy_(torch.rand(m.weight.shape, generator=g))
    f = lambda t: t.detach().float().cpu().numpy()
    gm, um, dm = model.layers[0].mlp.gate_proj, model.layers[0].mlp.up_proj, model.layers[0].mlp.down_proj
    ref = om.glu_joint_update(om.full_config(**kw), 3, f(gm.weight), f(gm.hessian_diag), f(gm.mask), f(um.weight),
                              f(um.hessian_diag), f(um.mask), None, None, 0.0)
    c = om.full_config(**kw)
    ref_d = om.layer_update_mask(c, 3, f(dm.weight), f(dm.hessian_diag), f(dm.mask), None, None, 0.0)
    U.calculate_model_mask(model, step=3)
    np.testing.assert_allclose(f(gm.mask), ref[0], rtol=0, atol=1e-6)
    np.testing.assert_allclose(f(um.mask), ref[1], rtol=0, atol=1e-6)
    np.testing.assert_allclose(f(dm.mask), ref_d[0], rtol=0, atol=1e-6)


def _layer(cfg_kw, W, H, M, tdt, dev, aux=None):
    sm = _sm()
    cfg = sm.SparseLinearConfig(**cfg_kw)
    cfg.enable_hutchinson = True
    layer = sm.SparseLinear(W.shape[1], W.shape[0], sparselinear_config=cfg, bias=False).to(tdt).to(dev)
    with torch.no_grad():
        layer.weight.copy_(torch.as_tensor(W).to(tdt))
        layer.hessian_diag.copy_(torch.as_tensor(H).to(tdt))
        layer.mask.copy_(torch.as_tensor(M).to(tdt))
    return layer


@pytest.mark.parametrize("metric", ["hessian_ratio", "hessian_obd", "hessian", "magnitude"])
@pytest.mark.parametrize("tdt", [torch.float32, torch.bfloat16])
def test_compute_importance_scores_bit_exact(cuda_device, metric, tdt):
    """utils._compute_importance_scores (legacy/utils.py:482-533) against oracle.masks.scores, bit for bit,
    with the reference's result dtype (ragged cols: a tail group)."""
    from sparseforge_amd import utils as U

    rng = np.random.default_rng(4)
    W = (rng.standard_normal((40, 70)) * 0.02).astype(np.float32)
    H = (rng.random((40, 70)) * 1e-3 + 1e-7).astype(np.float32)
    M = rng.random((40, 70)).astype(np.float32)
    layer = _layer(dict(mask_metric=metric), W, H, M, tdt, cuda_device)
    S = U._compute_importance_scores(layer)
    dt = F32 if tdt == torch.float32 else BF16
    Wd, Hd = (layer.weight.detach().float().cpu().numpy(), layer.hessian_diag.float().cpu().numpy())
    ref = om.scores(Wd, Hd, None, metric, dt, dt)
    assert S.dtype == tdt
    np.testing.assert_array_equal(S.float().cpu().numpy(), ref)


@pytest.mark.parametrize("tdt", [torch.float32, torch.bfloat16])
def test_compute_importance_scores_obd_without_hessian(cuda_device, tdt):
    """hessian_obd with hessian_diag left a placeholder scores W * W in W's dtype (legacy/utils.py:506-511),
    bit for bit (a product of two representable values rounds once).  A hessian_obd layer holds a full
    hessian_diag unless change_mask is off (legacy/sparse_modeling.py:318-334), so that is how the
    placeholder arises."""
    from sparseforge_amd import utils as U

    sm = _sm()
    cfg = sm.SparseLinearConfig(mask_metric="hessian_obd", change_mask=False)
    layer = sm.SparseLinear(70, 40, sparselinear_config=cfg, bias=False).to(tdt).to(cuda_device)
    assert layer._is_placeholder("hessian_diag")
    g = torch.Generator().manual_seed(2)
    with torch.no_grad():
        layer.weight.copy_((torch.randn(40, 70, generator=g) * 0.02).to(tdt))
    S = U._compute_importance_scores(layer)
    assert S.dtype == tdt
    W = layer.weight.detach().float().cpu().numpy()
    np.testing.assert_array_equal(S.float().cpu().numpy(), om.scores(W, None, None, "weight_squared",
                                                                      F32 if tdt == torch.float32 else BF16))


@pytest.mark.parametrize("kw", [dict(mask_type="unstructured"), dict(mask_type="structured"),
                                dict(mask_type="unstructured", beta_structural_start=0, beta_structural_end=10)])
@pytest.mark.parametrize("tdt", [torch.float32, torch.bfloat16])
def test_compute_joint_gate_target_matches_oracle(cuda_device, kw, tdt):
    """utils._compute_joint_gate_target (legacy/utils.py:536-613) on the summed scores of a gate/up pair,
    with frozen flags, against oracle.masks.joint_gate_target: within 1e-6 (f32) / one bf16 ulp."""
    from sparseforge_amd import utils as U

    rng = np.random.default_rng(9)
    shape = (64, 128)
    Wg, Wu = [(rng.standard_normal(shape) * 0.02).astype(np.float32) for _ in range(2)]
    Hg, Hu = [(rng.random(shape) * 1e-3 + 1e-6).astype(np.float32) for _ in range(2)]
    Mg = rng.random(shape).astype(np.float32)
    cfg_kw = dict(mask_metric="hessian_ratio", sparsity_warmup_steps=0, freeze_low=0.01, **kw)
    gate = _layer(cfg_kw, Wg, Hg, Mg, tdt, cuda_device)
    up = _layer(cfg_kw, Wu, Hu, Mg, tdt, cuda_device)
    F = (rng.random(shape) < 0.1).astype(np.float32)
    with torch.no_grad():
        gate.frozen_mask_flags.copy_(torch.as_tensor(F).to(tdt))
    S = U._compute_importance_scores(gate) + U._compute_importance_scores(up)
    idx = torch.as_tensor(rng.integers(0, S.numel(), 3000)).to(cuda_device)
    G = U._compute_joint_gate_target(gate, S, 7, sample_idx=idx)
    dt = F32 if tdt == torch.float32 else BF16
    ref = om.joint_gate_target(om.full_config(**cfg_kw), 7, S.float().cpu().numpy(), gate.mask.float().cpu().numpy(),
                               F, idx.cpu().numpy(), dt)
    assert G.dtype == tdt and G.shape == S.shape
    tol = 1e-6 if dt == F32 else 2 ** -8
    np.testing.assert_allclose(G.float().cpu().numpy(), ref, rtol=0, atol=tol)
    np.testing.assert_array_equal(G.float().cpu().numpy()[F > 0], gate.mask.float().cpu().numpy()[F > 0])
