"""The error bound of the Gram norm (oracle/ghost_oracle.py) -- CPU only.

The ghost norm ``S = <A A^T, G G^T>`` of an example cancels: its rounding error
scales with the Gram entries, not with ``||G^T A||^2``.  The device returns a
bound ``err`` with every squared norm and takes the clip factor from
``S + err``; the oracle restates that bound.  These tests pin it by its
defining property ``|S - ||G^T A||^2| <= err`` on fp32 accumulation chains
emulated with the two rounding behaviours the error model covers (to nearest
and truncation) on crafted cancellation inputs, with the exact float64 product
as the truth; they check that the DP guarantee ``c ||G^T A|| <= C`` then holds
with no tolerance, that planted mistakes (no bound, a chain unit 2^17 too
small) break it, and that the bound stays small on random data.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import clip_oracle, ghost_oracle


def _bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.bfloat16).double().numpy()


def _cancelling_example(T: int, d_in: int, d_out: int, ratio: float, seed: int):
    """Rows paired (t, t + T/2): equal activations, output gradients g + delta
    and -g with ||delta|| / ||g|| = ratio, so G^T A = sum_t delta_t a_t^T."""
    rng = np.random.default_rng(seed)
    h = T // 2
    a = _bf16(rng.standard_normal((h, d_in)))
    g = rng.standard_normal((h, d_out))
    delta = rng.standard_normal((h, d_out)) * ratio
    A = np.concatenate([a, a])
    G = _bf16(np.concatenate([g + delta, -g]))
    return A, G


def _exact_sq(A: np.ndarray, G: np.ndarray) -> float:
    w = G.T @ A  # float64; exact enough: bf16 products, short sums
    return float((w * w).sum())


def _device_like(A, G, mode, *, u=None):
    P = ghost_oracle.emulated_gram(A, mode=mode)
    Q = ghost_oracle.emulated_gram(G, mode=mode)
    if u is None:
        return ghost_oracle.gram_error_bound(P, Q, d_p=A.shape[1], d_q=G.shape[1])
    saved = ghost_oracle.U_MFMA
    ghost_oracle.U_MFMA = u
    try:
        return ghost_oracle.gram_error_bound(P, Q, d_p=A.shape[1], d_q=G.shape[1])
    finally:
        ghost_oracle.U_MFMA = saved


def _scale(sq_upper: float, C: float) -> float:
    """The guarded fixed-C scale for a bf16 4096 x 4096 weight (float32)."""
    roundoff = clip_oracle.norm_roundoff(torch.float32, torch.float64, 1,
                                         clip_oracle.reduction_terms([4096 * 4096]))
    ratio = torch.tensor([C / math.sqrt(max(sq_upper, 0.0))], dtype=torch.float64)
    s = clip_oracle.finalize_scale(ratio, torch.bfloat16, torch.float32, roundoff,
                                   clamp_to_one=True)
    return float(s.to(torch.float32)[0])


@pytest.mark.parametrize("mode", ["rn", "rz"])
@pytest.mark.parametrize("ratio", [1e-2, 1e-3])
@pytest.mark.parametrize("T,d_in,d_out", [(2, 4096, 4096), (256, 512, 1024)])
def test_bound_covers_cancellation(mode, ratio, T, d_in, d_out):
    A, G = _cancelling_example(T, d_in, d_out, ratio, seed=T + d_in)
    exact = _exact_sq(A, G)
    S, err = _device_like(A, G, mode)
    assert abs(S - exact) <= err, (S, exact, err)
    # The DP guarantee, no tolerance: the scale taken from S + err keeps the
    # exact per-example gradient inside C.
    for C in (1e-3 * math.sqrt(exact), math.sqrt(exact), 10 * math.sqrt(exact)):
        c = _scale(S + err, C)
        assert c * math.sqrt(exact) <= C


def test_planted_mistakes_break_the_guarantee():
    # Two tokens, equal activations, gradients g + delta and -g: the
    # configuration in which the unguarded Gram norm under-reports.
    violations_no_bound = 0
    violations_small_u = 0
    for seed in range(8):
        A, G = _cancelling_example(2, 4096, 4096, 1e-3, seed=100 + seed)
        exact = _exact_sq(A, G)
        S, _ = _device_like(A, G, "rz")
        C = 0.5 * math.sqrt(exact)  # clipping active
        # Planted mistake 1: no error term (the guard alone).
        if S <= 0 or _scale(S, C) * math.sqrt(exact) > C:
            violations_no_bound += 1
        # Planted mistake 2: a chain unit 2^17 too small -- a bound the size of
        # a typical accumulation error rather than the worst case.
        S2, err2 = _device_like(A, G, "rz", u=2.0 ** -40)
        if abs(S2 - exact) > err2:
            violations_small_u += 1
    assert violations_no_bound > 0
    assert violations_small_u > 0


def test_bound_is_tight_on_random_data():
    # Config-2 shapes (T = 512, d = 4096), N(0, 1) activations and gradients:
    # the bound inflates the squared norm by well under 2%.
    rng = np.random.default_rng(5)
    A = _bf16(rng.standard_normal((512, 4096)))
    G = _bf16(rng.standard_normal((512, 4096)) * 1e-5)
    S, err = _device_like(A, G, "rn")
    exact = _exact_sq(A, G)
    assert abs(S - exact) <= err
    assert err / exact < 2e-2, err / exact
    assert abs(S - exact) / exact < 1e-4


def test_generic_fp64_bound():
    # The generic kernels accumulate in fp64 (64-row tiles): the bound covers
    # a float64 chain on a cancelling example and is negligible on random data.
    A, G = _cancelling_example(70, 33, 65, 1e-6, seed=9)
    P, Q = A @ A.T, G @ G.T
    S, err = ghost_oracle.gram_error_bound(P, Q, d_p=33, d_q=65, tile=64, mfma=False)
    assert abs(S - _exact_sq(A, G)) <= err
    rng = np.random.default_rng(10)
    A, G = rng.standard_normal((130, 40)), rng.standard_normal((130, 72))
    S, err = ghost_oracle.gram_error_bound(A @ A.T, G @ G.T, d_p=40, d_q=72, tile=64,
                                           mfma=False)
    exact = _exact_sq(A, G)
    assert abs(S - exact) <= err
    assert err / exact < 1e-9


def test_chain_gamma_closed_form():
    # gamma(n) = g / (1 - g), g = 1.125 n u, rounded up by 2^-40.
    g = 1.125 * 4096 * 2.0 ** -23
    assert ghost_oracle.chain_gamma(4096, 2.0 ** -23) == pytest.approx(g / (1 - g), rel=1e-11)
    assert ghost_oracle.chain_gamma(4096, 2.0 ** -23) > g / (1 - g)
    assert math.isinf(ghost_oracle.chain_gamma(2.0 ** 22, 2.0 ** -23))
    # The row slack carries the flushed-subnormal term: eta <= gamma * slack^2.
    for n in (32, 4096, 1 << 20):
        assert n * 2.0 ** -125 <= ghost_oracle.chain_gamma(n, 2.0 ** -23) * 2.0 ** -102
