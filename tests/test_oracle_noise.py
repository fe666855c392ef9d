"""Pins of the key derivation and the noise oracle -- CPU only.

* key / fold_in / split: the properties the reference's RNG tests state
  (packages/opake-engine/tests/rng/test_rng_engine.py:19-101,
  test_stream_root_namespacing.py), checked on both the product's
  ``opake_amd.random`` and the oracle's restatement, and the two agree.
* reference-stream noise: the statistics of
  packages/opake-dpsgd/tests/noise/test_noise.py:112-139 (KS at p > 0.01 on
  10k draws, std within 0.1, realised RMS within 6 standard errors on 1e6),
  the per-group sigma values of :206-228 (4.0 and 6.928203230275509), and the
  draw order (dict keys sorted, one generator).
* Philox4x32-10 of the C oracle: the Random123 known-answer vectors; the
  device-stream Box-Muller map: distribution tests.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import scipy.stats
import torch

from opake_amd import random as rnd
from opake_amd.noise_allocation import (
    PAIRED_FIRST_STREAM_FOLD,
    PAIRED_SECOND_STREAM_FOLD,
    per_group_noise_stddev,
)
from opake_amd.types import PerGroup
from oracle import c_oracle, noise_oracle

RANDOM123_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


# --- keys ------------------------------------------------------------------------


def test_fold_in_chaining_and_split():
    k = rnd.key(42)
    assert rnd.fold_in(rnd.fold_in(k, 7), 3) == rnd.fold_in(k, 7, 3)
    assert rnd.fold_in(rnd.fold_in(rnd.fold_in(rnd.key(0), 1), 2), 3) == rnd.fold_in(rnd.key(0), 1, 2, 3)
    c = rnd.split(rnd.key(123), 3)
    assert len({x.seed for x in c}) == 3
    assert c == tuple(rnd.fold_in(rnd.key(123), i) for i in range(3))


def test_int_and_str_tags_are_disjoint():
    base = rnd.key(1234)
    for v in (0, 1, 2, 17):
        assert rnd.fold_in(base, v).seed != rnd.fold_in(base, str(v)).seed
    # Same 16 payload bytes, different tag byte.
    assert rnd.fold_in(rnd.key(42), 1).seed != rnd.fold_in(rnd.key(42), "\x01" + "\x00" * 15).seed


def test_key_validation():
    with pytest.raises(TypeError, match="seed must be int"):
        rnd.key("42")
    with pytest.raises(TypeError, match="seed must be int"):
        rnd.key(True)
    with pytest.raises(TypeError, match="int or str"):
        rnd.fold_in(rnd.key(1), True)
    with pytest.raises(TypeError, match="int or str"):
        rnd.fold_in(rnd.key(1), 1.5)
    with pytest.raises(ValueError, match="at least one data argument"):
        rnd.fold_in(rnd.key(1))
    with pytest.raises(TypeError, match="num must be int"):
        rnd.split(rnd.key(1), 2.0)
    assert rnd.key(-1).seed == (1 << 64) - 1


def test_stream_roots():
    assert PAIRED_FIRST_STREAM_FOLD == "opake.paired.first"
    assert PAIRED_SECOND_STREAM_FOLD == "opake.paired.second"
    base = rnd.key(42)
    reachable = {c.seed for c in rnd.split(base, 16)}
    reachable |= {rnd.fold_in(base, i).seed for i in range(512)}
    for tag in (PAIRED_FIRST_STREAM_FOLD, PAIRED_SECOND_STREAM_FOLD, noise_oracle.GAUSSIAN_STREAM_FOLD):
        assert rnd.fold_in(base, tag).seed not in reachable


def test_product_keys_match_oracle():
    for seed in (0, 1, 42, 2**63 + 5, (1 << 64) - 1):
        k = rnd.key(seed)
        for step in (0, 1, 99):
            want = noise_oracle.step_seed(noise_oracle.key_seed(seed), step)
            assert rnd.fold_in(k, "opake.dpsgd.gaussian", step).seed == want


def test_generator_from_key_reproducible_and_mod():
    k = rnd.key(999)
    assert torch.equal(torch.randn(16, generator=rnd.generator_from_key(k)),
                       torch.randn(16, generator=noise_oracle.generator_for(999)))
    big = rnd.key(2**63 - 1 + 5)  # reduced mod 2^63 - 1 -> 5
    assert torch.equal(torch.randn(4, generator=rnd.generator_from_key(big)),
                       torch.randn(4, generator=torch.Generator().manual_seed(5)))


# --- reference-stream noise ------------------------------------------------------


def _noised_zeros(n, nm, max_norm, seed):
    z = torch.zeros(n)
    s = noise_oracle.step_seed(noise_oracle.key_seed(seed), 0)
    draw = noise_oracle.draws_for([z], s)[0]
    return noise_oracle.sample(z, nm * max_norm, draw)


def test_noise_normality():
    out = _noised_zeros(10000, 1.0, 1.0, 42)
    _, p = scipy.stats.kstest(out.numpy(), scipy.stats.norm.cdf)
    assert p > 0.01


def test_noise_stddev():
    out = _noised_zeros(10000, 2.5, 1.0, 0)
    assert abs(out.std().item() - 2.5) < 0.1


def test_realised_stddev_matches_reported():
    std = 1.5 * 0.8
    out = _noised_zeros(1_000_000, 1.5, 0.8, 42).double()
    rms = out.pow(2).mean().sqrt().item()
    se = std / math.sqrt(2 * out.numel())
    assert abs(rms - std) < 6 * se
    assert abs(0.97 * rms - std) > 6 * se  # a 3% error is caught


def test_per_group_stddev_values():
    pg = PerGroup(groups={"w": "small", "b": "large"}, values={"small": 1.0, "large": 3.0})
    got = per_group_noise_stddev(pg, 2.0).values
    assert got["small"] == pytest.approx(4.0)
    assert got["large"] == pytest.approx(6.928203230275509)
    assert noise_oracle.per_group_noise_stddev({"small": 1.0, "large": 3.0}, 2.0) == pytest.approx(
        {"small": 4.0, "large": 6.928203230275509})
    assert per_group_noise_stddev(pg, 0.0).values == {"small": 0.0, "large": 0.0}


def test_draw_order_is_sorted_keys_one_generator():
    tree = {"weight": torch.zeros(3, 2), "bias": torch.zeros(3)}
    leaves = noise_oracle.flatten_sorted(tree)
    assert leaves[0].shape == (3,)
    gen = torch.Generator().manual_seed(7)
    b = torch.randn(3, generator=gen)
    w = torch.randn(3, 2, generator=gen)
    d = noise_oracle.draws_for(leaves, 7)
    assert torch.equal(d[0], b) and torch.equal(d[1], w)


def test_sample_rounds_once_back_to_bf16():
    c = torch.tensor([1.0, -2.0, 0.5], dtype=torch.bfloat16)
    z = torch.tensor([0.3, 0.7, -1.1])
    out = noise_oracle.sample(c, 0.25, z)
    assert out.dtype == torch.bfloat16
    assert torch.equal(out, (c.float() + 0.25 * z).to(torch.bfloat16))
    assert noise_oracle.sample(c, 0.0, z) is c


# --- Philox / device stream --------------------------------------------------------


@pytest.mark.parametrize("ctr,key,expected", RANDOM123_KAT)
def test_c_oracle_philox_known_answers(ctr, key, expected):
    got = c_oracle.philox(ctr, key, 1)[0]
    assert tuple(int(x) for x in got) == expected


def test_device_stream_distribution():
    z = c_oracle.leaf_normals(0x0123456789ABCDEF, 0, 1000, 200).ravel()
    _, p = scipy.stats.kstest(z, scipy.stats.norm.cdf)
    assert p > 1e-3
    assert abs(z.mean()) < 5 / math.sqrt(z.size)
    assert abs(z.var() - 1.0) < 5 * math.sqrt(2 / z.size)
    # Pairs from one block are uncorrelated.
    zz = c_oracle.leaf_normals(5, 1, 2, 100000)
    assert abs(np.corrcoef(zz[0], zz[1])[0, 1]) < 5 / math.sqrt(100000)


def test_device_stream_depends_on_seed_and_leaf():
    a = c_oracle.leaf_normals(1, 0, 4, 8)
    assert not np.array_equal(a, c_oracle.leaf_normals(2, 0, 4, 8))
    assert not np.array_equal(a, c_oracle.leaf_normals(1, 1, 4, 8))
    # Rows are paired: the first two rows of a [4, 8] leaf equal a [2, 8] leaf.
    assert np.array_equal(a[:2], c_oracle.leaf_normals(1, 0, 2, 8))
