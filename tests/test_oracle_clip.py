"""Pins of the CPU clipping oracle (oracle/clip_oracle.py) -- CPU only.

Each check is a closed form or invariant stated by the reference's own tests,
chosen so that a plausible restatement slip (a dropped guard term, the wrong
dtype in the multiply, a missing sanitise, clamping AUTO-S to 1) fails one:

* closed forms of packages/opake-engine/tests/clipping/test_clipped_fun.py:33-83
  and test_auto.py:24-62;
* the stored-value bound ``||stored|| <= C`` with no tolerance, for every dtype
  and magnitude (test_clipping_numerics.py:61-83,118-133);
* exact pass-through, exact zeros at C = 0, float32 guard ~1e-6, widened
  multiply (test_clipping_numerics.py:170-227);
* the boundary pin ``[[3,4],[0.6,0.8]], C=1 -> [1.2, 1.6]``
  (packages/opake-patches/tests/kernels/test_clip_sum.py:156-161).
"""

from __future__ import annotations

import math

import pytest
import torch

from opake_amd.clipping import _numerics as num
from oracle import clip_oracle as co

DTYPES = [torch.float16, torch.bfloat16, torch.float32, torch.float64]
MAGNITUDES = [1e-30, 1e-6, 1e-2, 1.0, 1e3, 1e20]


def exact_norm(leaves) -> float:
    return math.sqrt(sum(float((l.double() ** 2).sum()) for l in leaves))


# --- closed forms -----------------------------------------------------------


def test_clip_zero_returns_zeros_and_norm():
    out, norm = co.clip_pytree_scalar([torch.tensor([3.0, 4.0])], 0.0)
    assert torch.equal(out[0], torch.zeros(2))
    assert norm.item() == pytest.approx(5.0)


def test_clip_inf_is_passthrough():
    x = torch.tensor([3.0, 4.0])
    out, _ = co.clip_pytree_scalar([x], math.inf)
    assert torch.equal(out[0], x)


def test_clip_rescales_to_threshold():
    out, _ = co.clip_pytree_scalar([torch.tensor([3.0, 4.0])], 1.0)
    assert exact_norm(out) == pytest.approx(1.0, rel=1e-6)
    assert exact_norm(out) <= 1.0


def test_clip_below_threshold_unchanged():
    x = torch.tensor([0.3, 0.4])
    out, _ = co.clip_pytree_scalar([x], 1.0)
    assert torch.equal(out[0], x)


def test_clip_sanitises_nonfinite():
    out, norm = co.clip_pytree_scalar([torch.tensor([math.nan, math.inf, 1.0])], 1.0)
    assert torch.isfinite(out[0]).all()
    assert math.isfinite(norm.item())
    assert norm.item() == 1.0


def test_auto_s_formula():
    x = torch.tensor([3.0, 4.0])
    out, norm = co.auto_scale_scalar([x], 1.0, 0.01)
    torch.testing.assert_close(out[0], x * (1.0 / 5.01))
    assert norm.item() == pytest.approx(5.0)


def test_auto_s_is_not_clamped_to_one():
    # ||g|| = 0.5 < R: AUTO-S still rescales to R * g / (||g|| + gamma) > g.
    x = torch.tensor([0.3, 0.4])
    out, _ = co.auto_scale_scalar([x], 1.0, 0.01)
    assert exact_norm(out) > 0.5
    torch.testing.assert_close(out[0], x * (1.0 / 0.51))


def test_auto_s_zero_gradient():
    out, norm = co.auto_scale_scalar([torch.zeros(4)], 1.0, 0.01)
    assert torch.equal(out[0], torch.zeros(4))
    assert norm.item() == 0.0


def test_boundary_pin_from_reference_kernel_tests():
    batch = torch.tensor([[3.0, 4.0], [0.6, 0.8]])
    res = co.stream_clip_and_sum([batch], co.conservative_bound(1.0))
    torch.testing.assert_close(res.reduced[0], torch.tensor([1.2, 1.6]))
    # The example with ||g|| == C is still scaled by < 1 (guard before min(1, .)).
    assert res.scales[torch.float32][1].item() < 1.0


# --- invariants ---------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES)
def test_stored_bound_holds_exactly(dtype):
    gen = torch.Generator().manual_seed(0)
    for m in MAGNITUDES:
        for C in (0.01, 1.0, 7.5):
            leaves = [(torch.randn(33, generator=gen) * m).to(dtype),
                      (torch.randn(4, 5, generator=gen) * m).to(dtype)]
            out, _ = co.clip_pytree_scalar(leaves, C)
            assert exact_norm(out) <= C, (dtype, m, C)


@pytest.mark.parametrize("dtype", DTYPES)
def test_auto_s_stored_bound_holds_exactly(dtype):
    gen = torch.Generator().manual_seed(1)
    for m in MAGNITUDES:
        for R in (0.01, 1.0, 7.5):
            out, _ = co.auto_scale_scalar([(torch.randn(64, generator=gen) * m).to(dtype)], R, 0.01)
            assert exact_norm(out) <= R, (dtype, m, R)


@pytest.mark.parametrize("n_leaves", [1, 50, 200])
def test_bound_holds_as_leaf_count_grows(n_leaves):
    gen = torch.Generator().manual_seed(8)
    for _ in range(5):
        leaves = [(torch.randn(64, generator=gen, dtype=torch.float64) * 10).float()
                  for _ in range(n_leaves)]
        out, _ = co.clip_pytree_scalar(leaves, 1.0)
        assert exact_norm(out) <= 1.0


def test_without_guard_the_bound_fails():
    # Planted mistake (in the oracle, on the CPU): with rel = 1, abs = 0 the
    # stored bf16 norm exceeds C for some inputs, so the bound test above is
    # sensitive to the guard.
    gen = torch.Generator().manual_seed(0)
    violations = 0
    for _ in range(200):
        x = (torch.randn(64, generator=gen) * 10).to(torch.bfloat16)
        norm = math.sqrt(float((x.double() ** 2).sum()))
        stored = (x.float() * torch.tensor(1.0 / norm, dtype=torch.float32)).to(torch.bfloat16)
        violations += exact_norm([stored]) > 1.0
    assert violations > 0


@pytest.mark.parametrize("dtype", DTYPES)
def test_guard_does_not_perturb_unclipped(dtype):
    x = torch.tensor([0.03, -0.04], dtype=dtype)
    assert torch.equal(co.clip_pytree_scalar([x], 1000.0)[0][0], x)
    assert torch.equal(co.clip_pytree_scalar([x], math.inf)[0][0], x)
    z = torch.zeros(2, dtype=dtype)
    assert torch.equal(co.clip_pytree_scalar([z], 1.0)[0][0], z)


@pytest.mark.parametrize("dtype", DTYPES)
def test_zero_clipping_norm_exact_zeros(dtype):
    out, _ = co.clip_pytree_scalar([torch.tensor([3.0, 4.0], dtype=dtype)], 0.0)
    assert torch.equal(out[0], torch.zeros(2, dtype=dtype))


def test_guard_negligible_at_float32():
    out, _ = co.clip_pytree_scalar([torch.tensor([300.0, 400.0])], 1.0)
    assert exact_norm(out) == pytest.approx(1.0, rel=1e-6)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_low_precision_multiply_in_float32(dtype):
    ratio = torch.ones((), dtype=torch.float64)
    native = co.finalize_scale(ratio, dtype, dtype, 0.0, clamp_to_one=False)
    widened = co.finalize_scale(ratio, dtype, torch.float32, 0.0, clamp_to_one=False)
    assert widened > native
    leaf = torch.tensor([1.0, 0.5, -0.75], dtype=dtype)
    scaled = co.scale_tensor(leaf, ratio, torch.float32, 0.0, clamp_to_one=False)
    assert torch.equal(scaled, (leaf.float() * widened.float()).to(dtype))


def test_subnormal_rounded_up_goes_to_zero():
    quantum = torch.finfo(torch.float16).smallest_normal * torch.finfo(torch.float16).eps
    out, _ = co.clip_pytree_scalar([torch.tensor([2.0 ** -10], dtype=torch.float16)],
                                   0.5015 * quantum, compute_dtype=torch.float32)
    assert torch.equal(out[0], torch.zeros(1, dtype=torch.float16))


# --- guard constants: closed forms from torch.finfo ---------------------------


def test_guard_relative_constants():
    # bf16 leaves multiplied in fp32: rounding = eps_bf16 / 2 + eps_fp32.
    rel, absolute = co.guard_constants(torch.bfloat16, torch.float32, 0.0)
    assert rel == 1.0 - 2.0 ** -8 - 2.0 ** -23
    assert absolute == 2.0 ** -126 * 2.0 ** -7
    rel32, _ = co.guard_constants(torch.float32, torch.float32, 0.0)
    assert rel32 == 1.0 - 2.0 ** -23


def test_reduction_terms_and_roundoff():
    assert co.reduction_terms([1]) == 0
    assert co.reduction_terms([4096]) == 4096
    assert co.reduction_terms([4097]) == 2048 + 3
    # Config-2 weight leaf, 4096 x 4096 elements.
    n_red = co.reduction_terms([4096 * 4096])
    assert n_red == 2048 + 8192
    r = co.norm_roundoff(torch.float32, torch.float64, 1, n_red)
    assert r == pytest.approx((2.0 ** -24 + (1 + n_red) * 2.0 ** -53) / 2.0, rel=0, abs=0)


def test_product_numerics_match_oracle():
    # The host-side guard closed forms of the product agree with the oracle.
    for storage, mult in [(torch.bfloat16, torch.float32), (torch.float32, torch.float32),
                          (torch.float16, torch.float32), (torch.float64, torch.float64)]:
        for r in (0.0, 2.98e-8):
            assert num.guard_constants(storage, mult, r) == co.guard_constants(storage, mult, r)
    for sizes in ([1], [10], [4096], [4097, 3], [4096 * 4096, 4096]):
        assert num.reduction_terms(sizes) == co.reduction_terms(sizes)
    for C in (1.0, 0.1, 1e-3, 3.0, 0.35355339059327373):
        assert num.conservative_bound(C) == co.conservative_bound(C)
        assert num.conservative_bound(C) <= C


def test_conservative_bound_rounds_down():
    # float32(0.1) rounds up, so the bound moves one ulp down.
    b = co.conservative_bound(0.1)
    assert b < 0.1
    assert torch.tensor(b, dtype=torch.float32).item() == b


# --- streaming clip-and-sum vs per-example clip_pytree ------------------------


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_stream_equals_per_example_clip_then_sum(dtype):
    gen = torch.Generator().manual_seed(5)
    B = 6
    leaves = [(torch.randn(B, 3, 4, generator=gen) * torch.exp(torch.randn(B, 1, 1, generator=gen))
               ).to(dtype), (torch.randn(B, 7, generator=gen)).to(dtype)]
    res = co.stream_clip_and_sum(leaves, 1.0, return_aux=True)
    per = [co.clip_pytree_scalar([l[b] for l in leaves], 1.0)[0] for b in range(B)]
    for i in range(len(leaves)):
        acc = torch.float32 if dtype == torch.bfloat16 else None
        want = torch.stack([p[i] for p in per]).sum(0, dtype=acc).to(dtype)
        assert torch.equal(res.reduced[i], want)
    assert (res.clipped_norms <= 1.0 + 1e-6).all()


def test_stream_auto_s_and_nonfinite():
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(4, 10, generator=gen)
    x[2, 3] = math.nan
    res = co.stream_clip_and_sum([x], 1.0, kind="auto_s", gamma=0.01)
    xs = co.sanitize(x)
    n = xs.double().norm(dim=1)
    want = (xs * (1.0 / (n + 0.01)).float().unsqueeze(1)).sum(0)
    torch.testing.assert_close(res.reduced[0], want, rtol=1e-6, atol=1e-7)
    assert torch.isfinite(res.reduced[0]).all()


def test_second_moment_closed_form_and_per_example_identity():
    # [[3, 4], [0.6, 0.8]] with C = 1: both examples store ~[0.6, 0.8], so the
    # second moment is ~[0.72, 1.28]; it equals the sum of the squares of the
    # single-example clip (clip_pytree) of each example.
    x = torch.tensor([[3.0, 4.0], [0.6, 0.8]])
    res = co.stream_clip_and_sum([x], 1.0, second_moment=True)
    torch.testing.assert_close(res.squared[0], torch.tensor([0.72, 1.28]), rtol=1e-6, atol=0)
    g = torch.Generator().manual_seed(4)
    for dtype in (torch.float32, torch.bfloat16):
        leaves = [(torch.randn(5, 7, generator=g) * 3).to(dtype),
                  (torch.randn(5, 300, generator=g)).to(dtype)]
        res = co.stream_clip_and_sum(leaves, 2.0, second_moment=True)
        for i in range(2):
            want = torch.zeros(leaves[i].shape[1:], dtype=torch.float32)
            for b in range(5):
                one, _ = co.clip_pytree_scalar([l[b] for l in leaves], 2.0)
                want += one[i].square().float()
            torch.testing.assert_close(res.squared[i].float(), want.to(dtype).float(),
                                       rtol=1e-6 if dtype == torch.float32 else 1e-2, atol=0)
