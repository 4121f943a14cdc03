"""The sorted tau sample (oracle/masks.py sorted_sample_indices, the law sf_sample_indices_sorted draws).

The reference draws its tau sample with torch.randint(0, n, (m,)) (legacy/sparse_modeling.py:993) and
takes torch.quantile of the sampled scores, which does not depend on the sample's order.  The build draws
the same law in non-decreasing order from exponential spacings.  Pinned here, on the CPU, by what the
mathematics fixes rather than by the construction itself:
* the k-th smallest of m independent U(0, 1) has mean (k + 1) / (m + 1) and variance
  (k + 1)(m - k) / ((m + 1)^2 (m + 2)) (0-based k): over many seeds, every order statistic's sample mean
  stays within 5 standard errors (an off-by-one in the spacings, a wrong normaliser or a missing term
  moves the means by far more);
* every value of a tiny range is drawn with probability 1 / n (chi-square), so the floor and the clamp
  at n - 1 add no bias;
* the values of one long list pass a Kolmogorov-Smirnov test against the uniform law, as numpy's own
  uniform integers of the same size do.
"""
import numpy as np
import pytest

from oracle import masks as om


def test_sorted_and_in_range():
    for m, n, seed in ((1, 1, 0), (7, 3, 1), (1000, 17, 2), (4099, 1 << 24, 3), (262144, 45088768, 4)):
        idx = om.sorted_sample_indices(m, n, seed)
        assert idx.dtype == np.int64 and idx.shape == (m,)
        assert idx.min() >= 0 and idx.max() < n
        assert np.all(np.diff(idx) >= 0)


def test_order_statistics_moments():
    m, n, reps = 31, 1 << 40, 3000
    u = np.stack([om.sorted_sample_indices(m, n, 1000 + r) for r in range(reps)]).astype(np.float64) / n
    k = np.arange(m)
    mean = (k + 1) / (m + 1)
    var = (k + 1) * (m - k) / ((m + 1) ** 2 * (m + 2))
    z = (u.mean(0) - mean) / np.sqrt(var / reps)
    assert np.abs(z).max() < 5.0, z
    zv = (u.var(0) - var) / (var * np.sqrt(2.0 / reps))  # rough standard error of a variance
    assert np.abs(zv).max() < 6.0, zv


def test_tiny_range_frequencies():
    n, m = 5, 200000
    counts = np.bincount(om.sorted_sample_indices(m, n, 77), minlength=n)
    chi2 = float(((counts - m / n) ** 2 / (m / n)).sum())
    assert chi2 < 20.5, (counts, chi2)  # chi-square, 4 degrees of freedom: p = 4e-4
    assert counts[-1] > 0 and counts[0] > 0


def test_uniform_against_numpy():
    m, n = 262144, 45088768
    ks = lambda v: float(np.max(np.abs(np.sort(v) / n - (np.arange(1, v.size + 1) - 0.5) / v.size)))
    bound = 1.95 / np.sqrt(m)  # one-sample KS at p = 0.001
    assert ks(om.sorted_sample_indices(m, n, 9).astype(np.float64) + 0.5) < bound
    assert ks(np.random.default_rng(9).integers(0, n, m).astype(np.float64) + 0.5) < bound


def test_planted_off_by_one_fails():
    """A restatement that divides by S_(m-1) instead of S_m (the last draw then always lands at n - 1)
    fails the moment check: the check has teeth."""
    m, n, reps = 31, 1 << 40, 600

    def wrong(seed):
        from oracle.hutchinson import splitmix64

        j = np.arange(m + 1, dtype=np.uint64)
        r = splitmix64(seed, j) >> np.uint64(11)
        e = np.floor(-np.log((r.astype(np.float64) + 1.0) * 2.0 ** -53) * 2.0 ** 32 + 0.5).astype(np.uint64)
        s = np.cumsum(e, dtype=np.uint64)
        return np.minimum(np.floor(s[:m].astype(np.float64) / float(s[m - 1]) * n).astype(np.int64), n - 1)

    u = np.stack([wrong(1000 + r) for r in range(reps)]).astype(np.float64) / n
    k = np.arange(m)
    z = (u.mean(0) - (k + 1) / (m + 1)) / np.sqrt((k + 1) * (m - k) / ((m + 1) ** 2 * (m + 2)) / reps)
    assert np.abs(z).max() > 5.0


@pytest.mark.parametrize("m", [0, 5])
def test_small_lists(m):
    idx = om.sorted_sample_indices(m, 10, 3)
    assert idx.shape == (m,)
