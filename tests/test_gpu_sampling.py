"""The sorted tau sampler on the device (sf_sample_indices_sorted) against its oracle.

The law it draws (m uniform draws from [0, n) in non-decreasing order, the law of the reference's
torch.randint sample at legacy/sparse_modeling.py:993 up to order) is pinned on the CPU in
tests/test_oracle_sampling.py.  Bar: equal to oracle.masks.sorted_sample_indices index for index.  The
device and numpy logarithms are each within an ulp, so an E_j may round to a neighbouring 2^-32 step
once in about 2^19 draws; that moves later sums by one unit in 2^32 and an index only when it sits that
close to an integer, so at most a couple of indices may differ, by one.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _check(got, m, n, seed):
    from oracle import masks as om

    want = om.sorted_sample_indices(m, n, seed)
    d = np.abs(got.astype(np.int64) - want)
    assert int((d != 0).sum()) <= 2 and int(d.max(initial=0)) <= 1, (m, n, seed, int((d != 0).sum()))
    assert np.all(np.diff(got) >= 0) and got.min(initial=0) >= 0 and got.max(initial=0) < n


@pytest.mark.parametrize("m", [1, 5, 4095, 4096, 262144])
def test_sorted_sampler_matches_oracle(cuda_device, m):
    from sparseforge_amd import kernels as K

    ns = [1, 3, 16777216, 45088768]
    seeds = [11, 12, 2 ** 63 + 5, 99]
    rows = K.sample_indices_sorted(m, ns, seeds, cuda_device).cpu().numpy()
    for r, (n, s) in enumerate(zip(ns, seeds)):
        _check(rows[r], m, n, s)


def test_sorted_sampler_many_lists(cuda_device):
    """More lists than one launch carries (64): the launches split the lists and their workspace."""
    from sparseforge_amd import kernels as K

    ns = [1000 + 37 * c for c in range(150)]
    seeds = [c * 7919 for c in range(150)]
    rows = K.sample_indices_sorted(3000, ns, seeds, cuda_device).cpu().numpy()
    for c in (0, 63, 64, 127, 128, 149):
        _check(rows[c], 3000, ns[c], seeds[c])


def test_sorted_sampler_rejects_bad_calls(cuda_device):
    from sparseforge_amd import kernels as K

    with pytest.raises(ValueError):
        K.sample_indices_sorted(10, [0], [1], cuda_device)
    with pytest.raises(ValueError):
        K.sample_indices_sorted(10, [5, 6], [1], cuda_device)
    assert K.sample_indices_sorted(0, [5], [1], cuda_device).shape == (1, 0)
    assert K.sample_indices_sorted(5, [], [], cuda_device).shape == (0, 5)


def test_sorted_sampler_size_bound(cuda_device):
    """The largest sample the sorted path takes (2^28 - 1: 2^16 chunks of 4096 positions) is drawn sorted and
    in range; 2^28 is refused (the retraining code draws such samples with torch.randint instead)."""
    from sparseforge_amd import _lib as L
    from sparseforge_amd import kernels as K
    from sparseforge_amd import sparse_modeling as sm

    m, n = sm.SORTED_SAMPLE_MAX - 1, 45088768
    print(f"[sampling] size bound m={m}", flush=True)
    idx = K.sample_indices_sorted(m, [n], [11], cuda_device)[0]
    assert int(idx.min()) >= 0 and int(idx.max()) < n
    assert bool((idx[1:] >= idx[:-1]).all())
    # the mean of m uniform draws from [0, n) is (n - 1) / 2 within a few standard errors
    mean = float(idx.double().mean())
    assert abs(mean - (n - 1) / 2) < 6 * n / (12 * m) ** 0.5
    del idx
    big = torch.empty(1, dtype=torch.int64, device=cuda_device)
    ns = (L.ctypes.c_int64 * 1)(n)
    ss = (L.ctypes.c_uint64 * 1)(11)
    assert L.lib().sf_sample_indices_sorted(L.ptr(big), sm.SORTED_SAMPLE_MAX, ns, ss, 1, L.ptr(big), 1 << 20,
                                            L.stream(cuda_device)) == L.SF_ERR_INVALID
