"""Pins the block-sparse-16 oracle (oracle/bsr.py) on the CPU.

* Against the reference's own convert_to_block_sparse output
  (tests/golden/ref_bsr_basic_f32.npz): a fully pruned block, a zero inside a
  kept block, and a kept-by-mask block whose weights are all zero (dropped:
  the nonzero test uses W * mask, not the mask).
* Against a brute-force per-block scan on random masks, the NaN rule, the
  all-zero case, and the products against the dense masked matmul.
"""
import numpy as np
import pytest

from conftest import load_golden
from oracle import bsr as ob


def test_matches_reference_golden():
    r = load_golden("bsr_basic_f32")
    blocks, row_ptr, col_idx = ob.convert(r["W"], r["mask"], 16)
    assert np.array_equal(row_ptr, r["row_ptr"]) and np.array_equal(col_idx, r["col_idx"])
    assert np.array_equal(blocks, r["blocks"])


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_brute_force_and_products(seed):
    rng = np.random.default_rng(seed)
    W = rng.standard_normal((64, 96)).astype(np.float32)
    bm = rng.random((4, 6)) < 0.5
    M = np.kron(bm, np.ones((16, 16))).astype(np.float32)
    blocks, rp, ci = ob.convert(W, M)
    kept = [(r, c) for r in range(4) for c in range(6) if np.abs((W * M)[r * 16:(r + 1) * 16, c * 16:(c + 1) * 16]).sum() > 0]
    assert [(r, int(c)) for r in range(4) for c in ci[rp[r]:rp[r + 1]]] == kept
    assert np.array_equal(ob.to_dense(blocks, rp, ci, 64, 96), W * M)
    x = rng.standard_normal((10, 96))
    gy = rng.standard_normal((10, 64))
    np.testing.assert_allclose(ob.forward(x, blocks, rp, ci, 64, 96), x @ (W * M).T, rtol=1e-12)
    np.testing.assert_allclose(ob.input_grad(gy, blocks, rp, ci, 64, 96), gy @ (W * M), rtol=1e-12)
    dW = ob.sddmm_grad(gy, x, rp, ci)
    full = gy.T @ x
    for k, (r, c) in enumerate(kept):
        np.testing.assert_allclose(dW[k], full[r * 16:(r + 1) * 16, c * 16:(c + 1) * 16], rtol=1e-12)
    m = ob.block_map(rp, ci, 4, 6)
    assert ((m >= 0) == np.array([[(r, c) in kept for c in range(6)] for r in range(4)])).all()


def test_nan_block_dropped_and_all_zero():
    W = np.ones((32, 32), np.float32)
    W[3, 20] = np.nan
    blocks, rp, ci = ob.convert(W, np.ones_like(W))
    assert list(rp) == [0, 1, 3] and list(ci) == [0, 0, 1]  # block (0, 1) holds the NaN
    blocks, rp, ci = ob.convert(np.zeros((32, 48), np.float32), np.ones((32, 48), np.float32))
    assert blocks.shape == (1, 16, 16) and list(rp) == [0, 0, 0] and ci.size == 0


def test_flops():
    assert ob.flops(8192, 88064) == 2 * 8192 * 88064 * 256
