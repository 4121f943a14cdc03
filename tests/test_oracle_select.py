"""oracle.select (torch.topk's CPU selection restated) against torch.topk itself.

The block hard types and block penalty targets keep torch.topk's entries
(legacy/sparse_modeling.py:568, :649, :707, :1339, :1446, :1514); with equal
values which ones are kept is fixed by libstdc++'s nth_element / partial_sort
as torch calls them.  Tie-heavy inputs (a few distinct values), NaN and -0,
sizes on both sides of the k * 64 <= n partial-sort switch, and the two slice
shapes the reference uses (256-entry tiles and the flat block scores).
"""
import numpy as np
import pytest
import torch

from oracle import select as sel


def _torch_keep(v, k):
    return set(torch.topk(torch.from_numpy(v), k).indices.tolist())


@pytest.mark.parametrize("seed", range(6))
def test_topk_row_equals_torch_on_ties(seed):
    rng = np.random.default_rng(seed)
    for _ in range(120):
        n = int(rng.choice([1, 2, 3, 4, 5, 7, 16, 63, 64, 65, 256, 1000, 4099]))
        nv = int(rng.choice([1, 2, 3, 5, 50, 1 << 20]))
        v = (rng.integers(0, nv, size=n) / 7.0).astype(np.float32)
        if n > 3 and rng.random() < 0.3:
            v[rng.integers(0, n, size=2)] = np.nan
            v[rng.integers(0, n, size=2)] = -0.0
        for k in sorted({1, max(1, n // 64), max(1, n // 64 + 1), max(1, n // 2), max(1, n - 1), n}):
            assert set(sel.topk_row(v, k).tolist()) == _torch_keep(v, k), (n, nv, k)


def test_tiles_and_flat_scores_at_full_size():
    rng = np.random.default_rng(7)
    tiles = (rng.integers(0, 6, size=(500, 256)) / 5.0).astype(np.float32)
    for k in (1, 4, 5, 77, 128, 179, 255):
        got = sel.topk_keep(tiles, k)
        want = np.zeros_like(got)
        want[np.arange(500)[:, None], torch.topk(torch.from_numpy(tiles), k, dim=-1).indices.numpy()] = True
        assert np.array_equal(got, want), k
    flat = (rng.integers(0, 40, size=176128) / 7.0).astype(np.float32)
    flat[rng.integers(0, flat.size, size=5)] = np.nan
    for k in (88064, 1376, 2752, 176127):
        assert set(sel.topk_row(flat, k).tolist()) == _torch_keep(flat, k), k


def test_all_equal_and_degenerate_k():
    v = np.ones(256, np.float32)
    assert set(sel.topk_row(v, 128).tolist()) == _torch_keep(v, 128)
    assert sel.topk_row(v, 0).size == 0 and set(sel.topk_row(v, 256).tolist()) == set(range(256))
