"""Statistics of the on-GPU noise generator itself (GPU tests).

The device stream (Philox4x32-10 + Box-Muller) is a different stream from the
reference's CPU ``torch.randn`` with the same distribution, so it is checked
by the statistical tests of the reference's noise suite
(packages/opake-dpsgd/tests/noise/test_noise.py:112-139: KS normality,
realised standard deviation) -- here on the draws of ``dpc_add_noise`` itself
at the config-2 leaf size (4096 x 4096 = 16.8M normals, a float32 leaf so that
no storage rounding enters the statistics), copied back to the host:

* KS test against N(0, 1) on a 1e6 subsample: p > 0.01 (the reference's bar);
* mean, variance, skewness and excess kurtosis within 6 standard errors;
* tail counts |z| > 4 and |z| > 5 within 6 standard deviations of their
  binomial expectations (the 53-bit radius uniform reaches |z| ~ 8.6);
* near-zero correlation between the two members of a Box-Muller pair (rows
  2r and 2r + 1), between adjacent columns, between two leaves of one seed
  and between two seeds of one leaf (|r| < 6 / sqrt(n));
* sigma scaling: ``sigma * z`` realises sigma to within 6 standard errors.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import scipy.stats
import torch

from opake_amd import _native as nat
from opake_amd import ops

pytestmark = pytest.mark.gpu

ROWS = COLS = 4096
SEED = 0x0123_4567_89AB_CDEF


def _draw(dev, leaf_id=0, seed=SEED, sigma=1.0):
    zeros = torch.zeros(ROWS, COLS, dtype=torch.float32, device=dev)
    z = ops.add_noise(zeros, sigma, mode=nat.NOISE_PHILOX, seed=seed, leaf_id=leaf_id)
    return z.cpu().numpy().astype(np.float64)


@pytest.fixture(scope="module")
def z(dev):
    return _draw(dev)


def test_ks_normality(z):
    rng = np.random.default_rng(0)
    sample = rng.choice(z.reshape(-1), size=1_000_000, replace=False)
    _, p = scipy.stats.kstest(sample, scipy.stats.norm.cdf)
    assert p > 0.01, p


def test_moments(z):
    x = z.reshape(-1)
    n = x.size
    mean = x.mean()
    d = x - mean
    var = (d * d).mean()
    skew = (d ** 3).mean() / var ** 1.5
    kurt = (d ** 4).mean() / var ** 2 - 3.0
    assert abs(mean) < 6 / math.sqrt(n), mean
    assert abs(var - 1.0) < 6 * math.sqrt(2.0 / n), var
    assert abs(skew) < 6 * math.sqrt(6.0 / n), skew
    assert abs(kurt) < 6 * math.sqrt(24.0 / n), kurt


@pytest.mark.parametrize("t", [4.0, 5.0])
def test_tails(z, t):
    n = z.size
    p = 2 * scipy.stats.norm.sf(t)
    count = int((np.abs(z) > t).sum())
    expect = n * p
    assert abs(count - expect) < 6 * math.sqrt(n * p * (1 - p)) + 1, (count, expect)
    assert np.abs(z).max() < 8.7  # the largest radius the 53-bit uniform allows


def _corr(a, b):
    a = a.reshape(-1) - a.mean()
    b = b.reshape(-1) - b.mean()
    return float((a * b).sum() / math.sqrt((a * a).sum() * (b * b).sum()))


def test_pair_and_neighbour_correlation(z):
    lim = lambda n: 6 / math.sqrt(n)  # noqa: E731
    r_pair = _corr(z[0::2], z[1::2])  # the two normals of one Box-Muller pair
    assert abs(r_pair) < lim(z.size / 2), r_pair
    r_col = _corr(z[:, :-1], z[:, 1:])
    assert abs(r_col) < lim(z.size), r_col
    r_row = _corr(z[:-2], z[2:])  # consecutive pair blocks of one column
    assert abs(r_row) < lim(z.size), r_row
    # Squared values too (a radius shared by a pair must not leak).
    r_sq = _corr(z[0::2] ** 2, z[1::2] ** 2)
    assert abs(r_sq) < lim(z.size / 2), r_sq


def test_leaf_and_seed_independence(dev, z):
    other_leaf = _draw(dev, leaf_id=1)
    other_seed = _draw(dev, seed=SEED + 1)
    lim = 6 / math.sqrt(z.size)
    assert abs(_corr(z, other_leaf)) < lim
    assert abs(_corr(z, other_seed)) < lim
    assert not np.array_equal(z, other_leaf)


def test_sigma_scaling(dev, z):
    sigma = 2.5
    scaled = _draw(dev, sigma=sigma)
    # float32(sigma) * z, the epilogue's product, exactly.
    want = (np.float32(sigma) * z.astype(np.float32)).astype(np.float64)
    assert np.array_equal(scaled, want)
    n = scaled.size
    assert abs(scaled.std() - sigma) < 6 * sigma / math.sqrt(2 * n)
