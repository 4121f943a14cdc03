"""Pins the mask oracle (oracle/masks.py) — CPU only.

* top-N selection against torch.topk itself (the library the reference calls);
* hard projections against torch.topk + scatter restated with torch;
* quantile against torch.quantile;
* gate target / update_mask / GLU joint update against golden vectors the
  reference code wrote (tests/golden/make_reference_golden.py);
* closed-form invariants of the structured gate.
"""
import ast
import itertools

import numpy as np
import pytest
import torch

from conftest import load_golden
from oracle import masks as om
from oracle.numerics import BF16, F32, round_bf16


def torch_keep(x: np.ndarray, k: int) -> np.ndarray:
    t = torch.from_numpy(x)
    idx = torch.topk(t, k, dim=-1).indices
    return torch.zeros_like(t, dtype=torch.bool).scatter_(-1, idx, True).numpy()


@pytest.mark.parametrize("k", [1, 2, 3])
def test_topk_all_weak_orderings(k):
    pats = np.array(list(itertools.product(range(4), repeat=4)), dtype=np.float32)
    assert (om.topk_keep(pats, k) == torch_keep(pats, k)).all()


@pytest.mark.parametrize("k", [1, 2, 3])
def test_topk_random_ties_nan_and_signed_zero(k):
    rng = np.random.default_rng(k)
    vals = np.array([0.0, -0.0, 1.0, -1.0, np.nan, np.inf, 0.5], dtype=np.float32)
    x = vals[rng.integers(0, len(vals), size=(400, 37, 4))]
    assert (om.topk_keep(x, k) == torch_keep(x, k)).all()
    y = rng.integers(0, 3, size=(300, 50, 4)).astype(np.float32)
    assert (om.topk_keep(y, k) == torch_keep(y, k)).all()


def test_kth_largest_matches_topk_values():
    rng = np.random.default_rng(3)
    x = rng.integers(0, 4, size=(200, 30, 4)).astype(np.float32)
    x[0, 0, 1] = np.nan
    for k in (1, 2, 3):
        ref = torch.topk(torch.from_numpy(x), k, dim=-1).values[..., -1].numpy()
        got = om.kth_largest(x, k)
        assert np.array_equal(ref, got, equal_nan=True)


def test_all_ones_mask_keeps_columns_2_3():
    hard = om.hard_mask_from_soft(np.ones((3, 8), np.float32), "nm_2_4")
    assert (hard == np.tile([0, 0, 1, 1], (3, 2))).all()


@pytest.mark.parametrize("cols", [4, 66, 7, 3])
def test_nm_2_4_projection_matches_torch(cols):
    rng = np.random.default_rng(cols)
    soft = rng.integers(0, 5, size=(9, cols)).astype(np.float32) / 4
    full = (cols // 4) * 4
    ref = np.ones_like(soft)
    if full:
        ref[:, :full] = torch_keep(soft[:, :full].reshape(9, -1, 4), 2).reshape(9, full)
    assert (om.hard_mask_from_soft(soft, "nm_2_4") == ref).all()
    if full:
        assert (ref[:, :full].reshape(9, -1, 4).sum(-1) == 2).all()


def test_structured_requires_divisible_cols():
    with pytest.raises(ValueError):
        om.hard_mask_from_soft(np.ones((2, 6), np.float32), "structured")


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-8, 8, 100000)).astype(np.float32)
    x[:4] = [np.nan, np.inf, -np.inf, -0.0]
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(round_bf16(x), ref, equal_nan=True)


@pytest.mark.parametrize("q", [0.0, 0.3, 0.5, 0.777, 1.0])
def test_quantile_matches_torch(q):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(4097).astype(np.float32)
    assert om.quantile_linear(x, q) == torch.quantile(torch.from_numpy(x), q).item()


def test_structured_gate_invariants():
    rng = np.random.default_rng(5)
    z = rng.standard_normal((16, 32)).astype(np.float32)
    G = om.gate_target(z, F32, "structured", 0.5)
    g = G.reshape(16, 8, 4)
    zz = z.reshape(16, 8, 4)
    second = om.kth_largest(zz, 2)
    at_second = np.take_along_axis(g, np.argmax(zz == second[..., None], -1)[..., None], -1)
    assert (at_second == 0.5).all()
    assert ((g > 0) & (g < 1)).all()
    assert ((g >= 0.5).sum(-1) >= 2).all()


def _dt(name):
    return BF16 if "bfloat16" in str(name) else F32


def _cfg(rec):
    return om.full_config(**ast.literal_eval(str(rec["cfg"])))


@pytest.mark.parametrize("case", ["gate_unstr_ratio_f32", "gate_unstr_beta_f32", "gate_unstr_frozen_f32",
                                  "gate_struct_f32", "gate_struct_exact_f32", "gate_unstr_ratio_bf16",
                                  "gate_struct_bf16", "gate_obd_noH_f32", "gate_obd_noH_bf16"])
def test_gate_target_matches_reference_golden(case):
    r = load_golden(case)
    c = _cfg(r)
    dt = _dt(r["dtype"])
    step = int(r["step"])
    sch = om.layer_schedule(c, step)
    assert sch["T"] == float(r["T"]) and sch["sparsity"] == float(r["sparsity"]) and sch["beta_s"] == float(r["beta_s"])
    frozen = r["frozen"] if r["frozen"].shape == r["W"].shape else None
    G = om.layer_gate_target(c, step, r["W"], r["H"], r["mask"], frozen, r["idx"], dt, dt, dt)
    tol = 1e-6 if dt == F32 else 2 ** -8
    np.testing.assert_allclose(G, r["G"], rtol=0, atol=tol)


@pytest.mark.parametrize("case", ["update_paper_f32", "update_mid_bin_f32", "update_struct_topn_f32",
                                  "update_freeze_f32", "update_paper_bf16", "update_obd_noH_f32"])
def test_update_mask_matches_reference_golden(case):
    r = load_golden(case)
    c = _cfg(r)
    dt = _dt(r["dtype"])
    mask = r["init_mask"].copy()
    frozen = r["init_frozen"].copy() if r["init_frozen"].shape == r["W"].shape else None
    for j, step in enumerate(r["steps"]):
        out = om.layer_update_mask(c, int(step), r["W"], r["H"], mask, frozen, r[f"idx{j}"], float(r["lam"]), dt, dt, dt)
        assert out is not None
        mask, nf, flips, hx = out
        if nf is not None:
            frozen = nf
        tol = 1e-6 if dt == F32 else 2 ** -8
        np.testing.assert_allclose(mask, r[f"mask{j}"], rtol=0, atol=tol)
        if frozen is not None:
            assert (frozen == r[f"frozen{j}"]).all()
        assert flips == int(r[f"flips{j}"])
        assert hx == float(r[f"hx{j}"])
        mask = r[f"mask{j}"].copy()  # continue from the reference state


def test_glu_joint_matches_reference_golden():
    """_update_glu_joint_mask (legacy/utils.py:363-479) on a gate/up pair, three consecutive steps."""
    r = load_golden("glu_joint_f32")
    c = om.full_config(**ast.literal_eval(str(r["cfg"])))
    Mg, Mu = r["init_Mg"], r["init_Mu"]
    for j, step in enumerate((1, 2, 3)):
        out = om.glu_joint_update(c, step, r["Wg"], r["Hg"], Mg, r["Wu"], r["Hu"], Mu, None, r[f"idx{j}"], 0.05)
        ng, nu, fg, fu, hx = out
        np.testing.assert_allclose(ng, r[f"Mg{j}"], rtol=0, atol=1e-6)
        np.testing.assert_allclose(nu, r[f"Mu{j}"], rtol=0, atol=1e-6)
        assert (fg, fu) == (int(r[f"flips_g{j}"]), int(r[f"flips_u{j}"]))
        assert hx == float(r[f"hx{j}"])
        Mg, Mu = r[f"Mg{j}"], r[f"Mu{j}"]


def test_glu_joint_same_target_for_both_masks():
    """Both masks move toward one G: with equal starting masks they stay equal, and the update of
    either mask equals a single-layer EMA toward that G."""
    rng = np.random.default_rng(4)
    W1, W2 = rng.standard_normal((8, 16), dtype=np.float32), rng.standard_normal((8, 16), dtype=np.float32)
    H1, H2 = rng.random((8, 16), dtype=np.float32), rng.random((8, 16), dtype=np.float32)
    M = rng.random((8, 16), dtype=np.float32)
    c = om.full_config(mask_type="structured", mask_metric="hessian_obd", sparsity_warmup_steps=0,
                       mask_update_period=1, mask_lr=0.2)
    ng, nu, _, _, _ = om.glu_joint_update(c, 5, W1, H1, M, W2, H2, M.copy(), None, None, 0.0)
    assert np.array_equal(ng, nu)
    G = (ng - np.float32(0.8) * M) / np.float32(0.2)  # EMA inverted: G is a structured sigmoid target
    gg = G.reshape(8, 4, 4)
    assert (np.abs(np.sort(gg, axis=-1)[..., 2] - 0.5) < 1e-5).all()  # the 2nd largest of each group sits at 0.5


# ---------------------------------------------------------------------------
# block hard types, block_sparse gate, block penalties (sparse_modeling.py:460-507, :537-718,
# :1100-1158, :1237, :1298-1529, :1598-1601)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["hardblk_block16_f32", "hardblk_block16_sr03_f32", "hardblk_block16_ones_f32",
                                  "hardblk_bs16_f32", "hardblk_bs16_sr03_f32", "hardblk_bs16_ones_f32",
                                  "hardblk_bs32_f32"])
def test_block_hard_masks_match_reference_golden(case):
    r = load_golden(case)
    got = om.hard_mask_from_soft(r["soft"], str(r["hard_type"]), sparsity_ratio=float(r["sr"]))
    assert np.array_equal(got, r["hard"])


def test_block_topk_matches_torch_on_distinct_values():
    """Global / per-tile top-k against torch.topk + scatter where no two values are equal."""
    rng = np.random.default_rng(11)
    v = rng.permutation(5000).astype(np.float32).reshape(10, 500) / 7.0
    for k in (0, 1, 17, 250, 499, 500):
        assert np.array_equal(om.topk_keep_desc(v, k), torch_keep(v, k) if 0 < k else np.zeros_like(v, bool))


def test_block_rms_and_mean_closed_forms():
    """Constant blocks give exactly their value (mean) and |value| (RMS); a block of +-a gives a."""
    x = np.zeros((32, 48), np.float32)
    x[:16, :16] = 0.3
    x[16:, 16:32] = -0.7
    x[:16, 32:] = np.where((np.indices((16, 16)).sum(0) % 2) == 0, 0.25, -0.25)
    m = om.block_mean(x, 16)
    r = om.block_rms(x, 16)
    assert m[0, 0] == np.float32(0.3) and m[1, 1] == np.float32(-0.7) and m[0, 2] == 0.0
    assert r[0, 0] == np.sqrt(np.float32(0.3) * np.float32(0.3)) and r[1, 1] == np.float32(0.7)
    assert r[0, 2] == np.float32(0.25) and r[1, 0] == 0.0
    b = om.blockify(x, "block_sparse16", F32)
    assert (b[:16, :16] == np.float32(0.3)).all() and (b[:16, 32:] == 0.0).all()


def test_block16_keeps_exact_count_per_tile():
    rng = np.random.default_rng(3)
    soft = rng.random((48, 40)).astype(np.float32)
    for sr, k in ((0.5, 128), (0.25, 192), (0.3, 179), (1.0, 0)):
        h = om.hard_mask_from_soft(soft, "block16", sparsity_ratio=sr)
        tiles = om.block_tiles(h, 16)
        assert (tiles.sum(-1) == k).all()
        assert (h[:, 32:] == 1).all() and (h[48:] == 1).all()
        # each kept element is >= every dropped element of its tile
        s = om.block_tiles(soft, 16)
        kept = np.where(tiles > 0, s, np.inf).min(-1)
        dropped = np.where(tiles > 0, -np.inf, s).max(-1)
        assert (kept >= dropped).all()


@pytest.mark.parametrize("case", ["gateblk_bs16_f32", "gateblk_bs32_struct_f32", "gateblk_bs16_small_f32"])
def test_block_gate_matches_reference_golden(case):
    r = load_golden(case)
    c = _cfg(r)
    step = int(r["step"])
    sch = om.layer_schedule(c, step)
    assert sch["T"] == float(r["T"]) and sch["sparsity"] == float(r["sparsity"])
    frozen = r["frozen"] if r["frozen"].shape == r["W"].shape else None
    G = om.layer_gate_target(c, step, r["W"], r["H"], r["mask"], frozen, r["idx"])
    np.testing.assert_allclose(G, r["G"], rtol=0, atol=1e-6)


@pytest.mark.parametrize("case", ["updblk_bs16_f32", "updblk_block16_pen_f32", "updblk_bs32_freeze_f32",
                                  "updblk_block16_hard_f32"])
def test_block_update_matches_reference_golden(case):
    r = load_golden(case)
    c = _cfg(r)
    mask = r["init_mask"].copy()
    frozen = r["init_frozen"].copy() if r["init_frozen"].shape == r["W"].shape else None
    for j, step in enumerate(r["steps"]):
        out = om.layer_update_mask(c, int(step), r["W"], r["H"], mask, frozen, r[f"idx{j}"], float(r["lam"]))
        assert out is not None
        mask, nf, flips, hx = out
        if nf is not None:
            frozen = nf
        np.testing.assert_allclose(mask, r[f"mask{j}"], rtol=0, atol=1e-6)
        if frozen is not None:
            assert (frozen == r[f"frozen{j}"]).all()
        assert flips == int(r[f"flips{j}"])
        assert hx == float(r[f"hx{j}"])
        mask = r[f"mask{j}"].copy()


@pytest.mark.parametrize("kw", [dict(mask_type="unstructured"), dict(mask_type="structured"),
                                dict(mask_type="unstructured", beta_structural_start=0, beta_structural_end=10),
                                dict(mask_type="structured", structured_exact=True)])
def test_joint_gate_target_on_a_layers_own_scores_is_its_gate_target(kw):
    """_compute_joint_gate_target(module, _compute_importance_scores(module), step) is
    compute_gate_target(step) for an f32 layer (utils.py:482-613 vs sparse_modeling.py:1018-1239), which
    the reference's own gate goldens pin; with frozen flags the override copies the current mask."""
    rng = np.random.default_rng(11)
    W = (rng.standard_normal((48, 64)) * 0.02).astype(np.float32)
    H = (rng.random((48, 64)) * 1e-3 + 1e-6).astype(np.float32)
    M = rng.random((48, 64)).astype(np.float32)
    F = (rng.random((48, 64)) < 0.1).astype(np.float32)
    idx = rng.integers(0, W.size, 500)
    c = om.full_config(mask_metric="hessian_ratio", sparsity_warmup_steps=0, **kw)
    S = om.scores(W, H, None, "hessian_ratio")
    for frozen in (None, F):
        a = om.joint_gate_target(c, 7, S, M, frozen, idx)
        b = om.layer_gate_target(c, 7, W, H, M, frozen, idx)
        np.testing.assert_array_equal(a, b)
        if frozen is not None:
            np.testing.assert_array_equal(a[F > 0], M[F > 0])
