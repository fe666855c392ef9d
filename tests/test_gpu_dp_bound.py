"""The DP guarantee of the ghost clip on the GPU (called through the C ABI).

The Gram norm ``S = <A A^T, G G^T>`` cancels, so every Gram kernel returns an
upper bound ``err`` of its rounding error and the clip factor is taken from
``S + err``.  These tests check, with no tolerance:

* ``|S - ||G_i^T A_i||^2| <= err`` for the dense MFMA, generic (fp32) and
  grouped kernels on random data and on crafted cancellation inputs (tokens in
  pairs with equal activations and output gradients ``g + delta`` and ``-g``,
  ``||delta|| / ||g||`` of 1e-2 and 1e-3), the exact float64 product as truth;
* ``scale_i ||G_i^T A_i||_fp64 <= C`` for every example the clip factors
  produce from them (fixed C and AUTO-S);
* that the clipped sums apply those scales without rounding an operand: the
  dense fast list, the slow list (G times the power of two of the scale, the
  mantissa on the accumulators), the grouped kernel and the generic kernel
  all agree with the exact float64 sum of ``c_i G_i^T A_i`` to within fp32
  accumulation (1e-5 relative on random data);

and that the bound is small on random data (well under 2% of ``S``).
"""

from __future__ import annotations

import math

import pytest
import torch

from opake_amd import _native as nat
from opake_amd import ops
from opake_amd.clipping import _numerics as num
from opake_amd.clipping import ghost_clip_sum, guard_for_linear
from oracle import ghost_oracle

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _cancelling(B, T, din, dout, ratio, dtype, gen):
    """B examples of T tokens in pairs (t, t + T/2): equal activations,
    output gradients g + delta and -g with ||delta|| / ||g|| = ratio."""
    h = T // 2
    a = torch.randn(B, h, din, generator=gen)
    g = torch.randn(B, h, dout, generator=gen)
    delta = torch.randn(B, h, dout, generator=gen) * ratio
    A = torch.cat([a, a], dim=1).to(dtype)
    G = torch.cat([g + delta, -g], dim=1).to(dtype)
    return A, G


def _exact_sq(A, G):
    w = torch.einsum("btm,btn->bmn", G.double(), A.double())
    return (w * w).sum(dim=(1, 2))


@pytest.mark.parametrize("dtype,T,din,dout", [
    (torch.bfloat16, 128, 256, 512),   # MFMA kernel, one tile
    (torch.bfloat16, 300, 64, 1024),   # MFMA kernel, 3 tiles, ragged, d_in < d_out
    (torch.bfloat16, 256, 1024, 64),   # MFMA kernel, operands swapped
    (torch.bfloat16, 512, 256, 256),   # MFMA, one operand per item (diagonal + off-diagonal sets)
    (torch.bfloat16, 200, 96, 96),     # MFMA, one operand per item, ragged second block
    (torch.float32, 130, 72, 40),      # generic kernel (fp64 accumulation)
    (torch.bfloat16, 70, 36, 20),      # generic kernel, misaligned widths
])
@pytest.mark.parametrize("ratio", [None, 1e-2, 1e-3])
def test_gram_error_bound_holds(dev, dtype, T, din, dout, ratio):
    gen = _gen(T + din + dout)
    if ratio is None:
        A = torch.randn(3, T, din, generator=gen).to(dtype)
        G = (torch.randn(3, T, dout, generator=gen) * 0.01).to(dtype)
    else:
        A, G = _cancelling(3, T, din, dout, ratio, dtype, gen)
    sq, err = ops.gram_sqnorms(A.to(dev), G.to(dev), return_error=True)
    sq, err = sq.cpu(), err.cpu()
    exact = _exact_sq(A, G)
    assert torch.all((sq - exact).abs() <= err), (sq, exact, err)
    assert torch.all(err >= 0)
    if ratio is None:
        assert torch.all(err / exact < 2e-2), err / exact


def _spread(shape, lo_exp, gen):
    """bf16 values whose magnitudes alternate between ~2^15 and ~2^lo_exp
    along the feature (K) dimension, each with a random sign: inside every
    16-product K block of an MFMA the addends then span 2^30 to 2^(2 lo_exp),
    where the alignment and truncation of the hardware adder, and (for
    lo_exp = -70) the flush of subnormal products, lose the most."""
    mant = 1.0 + torch.rand(shape, generator=gen)
    k = torch.arange(shape[-1])
    exp = torch.where(k % 2 == 0, 15.0, float(lo_exp))
    sign = torch.where(torch.rand(shape, generator=gen) < 0.5, -1.0, 1.0)
    return (sign * mant * torch.exp2(exp)).to(torch.bfloat16)


@pytest.mark.parametrize("lo_exp", [-15, -70])
@pytest.mark.parametrize("T,din,dout", [
    (512, 256, 256),   # one operand per work item (split kernel)
    (384, 128, 256),   # paired kernel (odd number of 128-row blocks)
    (70, 40, 24),      # generic kernel (misaligned widths)
])
def test_gram_error_bound_holds_on_exponent_spread(dev, lo_exp, T, din, dout):
    gen = _gen(T + din - lo_exp)
    A = _spread((2, T, din), lo_exp, gen)
    G = _spread((2, T, dout), lo_exp, gen)
    sq, err = ops.gram_sqnorms(A.to(dev), G.to(dev), return_error=True)
    sq, err = sq.cpu(), err.cpu()
    exact = _exact_sq(A, G)
    assert torch.all(torch.isfinite(sq)) and torch.all(err > 0)
    assert torch.all((sq - exact).abs() <= err), ((sq - exact).abs() / err)


def test_gram_error_bound_matches_oracle_formula(dev):
    # The device bound from its own fp32 Gram tiles against the oracle's
    # formula evaluated on the exact Gram matrices: the same up to the tiles'
    # rounding (and the dense kernel's tile order).
    gen = _gen(3)
    B, T, din, dout = 2, 300, 256, 512
    A = torch.randn(B, T, din, generator=gen).to(torch.bfloat16)
    G = (torch.randn(B, T, dout, generator=gen) * 0.1).to(torch.bfloat16)
    _, err = ops.gram_sqnorms(A.to(dev), G.to(dev), return_error=True)
    for b in range(B):
        Ad, Gd = A[b].double().numpy(), G[b].double().numpy()
        _, want = ghost_oracle.gram_error_bound(Ad @ Ad.T, Gd @ Gd.T, d_p=din, d_q=dout)
        assert err[b].item() == pytest.approx(want, rel=1e-3)


def test_gram_error_bound_matches_oracle_formula_split_items(dev):
    # As above for the kernel that computes one operand per work item (din ==
    # dout, an even number of 128-row blocks), whose diagonal tiles come from
    # their upper-triangular 32 x 32 blocks.
    gen = _gen(4)
    B, T, d = 2, 512, 192
    A = torch.randn(B, T, d, generator=gen).to(torch.bfloat16)
    G = (torch.randn(B, T, d, generator=gen) * 0.1).to(torch.bfloat16)
    sq, err = ops.gram_sqnorms(A.to(dev), G.to(dev), return_error=True)
    torch.testing.assert_close(sq.cpu(), _exact_sq(A, G), rtol=1e-4, atol=0)
    for b in range(B):
        Ad, Gd = A[b].double().numpy(), G[b].double().numpy()
        _, want = ghost_oracle.gram_error_bound(Ad @ Ad.T, Gd @ Gd.T, d_p=d, d_q=d)
        assert err[b].item() == pytest.approx(want, rel=1e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("ratio", [1e-2, 1e-3])
@pytest.mark.parametrize("auto_s", [None, 0.01])
def test_ghost_clip_is_dp_sound_on_cancellation(dev, dtype, ratio, auto_s):
    # T = 128: the bf16 clipped sum takes the MFMA kernel (T % 64 == 0).
    gen = _gen(int(1 / ratio) + (dtype == torch.float32))
    B, T, din, dout = 4, 128, 512, 256
    A, G = _cancelling(B, T, din, dout, ratio, dtype, gen)
    exact = _exact_sq(A, G).sqrt()
    for C in (0.25 * exact.min().item(), exact.median().item()):
        res, aux = ghost_clip_sum(A.to(dev), G.to(dev), clipping_norm=C, return_aux=True,
                                  auto_s_gamma=auto_s, dtype=torch.float32)
        scale = aux.clip_scales.cpu().double()
        bound = C if auto_s is None else C
        assert torch.all(scale * exact <= bound), (scale * exact / bound)
        assert torch.isfinite(res.pytree["weight"]).all()


def _clip(dev, A, G, C, err=True):
    B, T, din, dout = A.shape[0], A.shape[1], A.shape[2], G.shape[2]
    sq, e = ops.gram_sqnorms(A.to(dev), G.to(dev), return_error=True)
    cf = ops.clip_factors(sq, num.conservative_bound(C), [guard_for_linear(A.dtype, din, dout,
                                                                           False)],
                          err=e if err else None, count_threshold=num.float32_of(C))
    return cf


def _exact_sum(A, G, scale):
    return torch.einsum("b,btm,btn->mn", scale.double(), G.double(), A.double())


def _rel(got, want):
    got, want = got.double().cpu(), want.double().cpu()
    return ((got - want).norm() / want.norm().clamp_min(1e-300)).item()


@pytest.mark.parametrize("case", ["fast", "tiny_scale", "large_bc", "generic_fp32",
                                  "generic_bf16"])
def test_clipped_sum_applies_scales_exactly(dev, case):
    gen = _gen(41)
    B, T, din, dout = 5, 128, 256, 264
    dtype = torch.float32 if case == "generic_fp32" else torch.bfloat16
    if case == "generic_bf16":
        T = 100  # T % 64 != 0: generic kernel, chunks cut at example boundaries
    A = torch.randn(B, T, din, generator=gen)
    G = torch.randn(B, T, dout, generator=gen) * 0.01 * torch.exp(
        torch.randn(B, 1, 1, generator=gen))
    C = 1.0
    if case == "tiny_scale":
        G[1] *= 1e19  # scale < 2^-64: the plan's slow list
        G[3] *= 3e19
    elif case == "large_bc":
        C = 1e17  # B * C > 2^55: every example on the slow list
    A, G = A.to(dtype), G.to(dtype)
    cf = _clip(dev, A, G, C)
    plan = cf.plan[0].cpu().view(torch.int32)
    if case == "tiny_scale":
        assert int(plan[0]) == B and int(plan[1]) == B - 2
    if case == "large_bc":
        assert int(plan[0]) == B and int(plan[1]) == 0
    w, _ = ops.clipped_sum(A.to(dev), G.to(dev), cf.scale[0], plan=cf.plan[0],
                           out_dtype=torch.float32)
    want = _exact_sum(A, G, cf.scale[0].cpu())
    assert _rel(w, want) < 1e-5


def test_grouped_bound_and_exact_scaling(dev):
    gen = _gen(55)
    lengths = [[0, 1, 63, 64, 130], [128, 0, 200, 7, 64]]
    din, dout = 264, 136
    As, Gs = [], []
    for e, lens in enumerate(lengths):
        rows = sum(lens)
        As.append(torch.randn(rows, din, generator=gen).to(torch.bfloat16))
        G = torch.randn(rows, dout, generator=gen) * 0.05
        if e == 1:
            # Segment 2 (200 rows): pairs of rows that cancel.
            r0 = 128
            half = 100
            As[1][r0 + half:r0 + 2 * half] = As[1][r0:r0 + half]
            G[r0 + half:r0 + 2 * half] = -G[r0:r0 + half]
            G[r0:r0 + half] += torch.randn(half, dout, generator=gen) * 0.05 * 1e-3
        Gs.append(G.to(torch.bfloat16))
    layout = ops.SegmentLayout(lengths, dev)
    seg_sq, seg_err = ops.grouped_gram_sqnorms([a.to(dev) for a in As], [g.to(dev) for g in Gs],
                                               layout, return_error=True)
    for e, lens in enumerate(lengths):
        want = (ghost_oracle.segment_grads(As[e], Gs[e], lens, dtype=torch.float64) ** 2).sum(
            dim=(1, 2))
        for k in range(len(lens)):
            assert abs(seg_sq[e, k].item() - want[k].item()) <= seg_err[e, k].item(), (e, k)
    scale = torch.rand(len(lengths), len(lengths[0]), generator=gen) * 3.0 + 1e-3
    scale[0, 2] = 2.0 ** -70  # any positive scale: the power of two goes to G
    out = ops.grouped_clipped_sum([a.to(dev) for a in As], [g.to(dev) for g in Gs], layout,
                                  scale.to(dev), out_dtype=torch.float32)
    for e, lens in enumerate(lengths):
        grads = ghost_oracle.segment_grads(As[e], Gs[e], lens, dtype=torch.float64)
        want = sum(scale[e, k].double() * grads[k] for k in range(len(lens)))
        assert _rel(out[e], want) < 1e-5, e


@pytest.mark.parametrize("case", ["fast", "split_k", "slow"])
def test_ghost_clip_sum_auto_s_matches_oracle(dev, case):
    # AUTO-S scales C / (||g|| + gamma) exceed 1 for small gradients; scales
    # above 2^32 go to the plan's slow list.
    from oracle import clip_oracle

    gen = _gen(71)
    B, T, din, dout = (6, 128, 256, 256) if case != "split_k" else (16, 128, 256, 256)
    A = torch.randn(B, T, din, generator=gen)
    G = torch.randn(B, T, dout, generator=gen) * 0.01 * torch.exp(
        torch.randn(B, 1, 1, generator=gen))
    gamma = 0.01 if case != "slow" else 1e-12
    if case == "slow":
        G[2] *= 1e-13  # ||g|| ~ 1e-12: scale ~ C / 2e-12 > 2^32
    A, G = A.to(torch.bfloat16), G.to(torch.bfloat16)
    res, aux = ghost_clip_sum(A.to(dev), G.to(dev), clipping_norm=1.0, auto_s_gamma=gamma,
                              return_aux=True, dtype=torch.float32)
    scale = aux.clip_scales.cpu()
    if case == "slow":
        assert scale[2].item() > 2.0 ** 32
    want = _exact_sum(A, G, scale)
    assert _rel(res.pytree["weight"], want) < 1e-5
    # Against the materialised oracle (AUTO-S on the rounded per-example
    # gradients): the bf16 tolerance.
    leaves = ghost_oracle.linear_per_example_grads(A, G)
    ref = clip_oracle.stream_clip_and_sum(leaves, clip_oracle.conservative_bound(1.0),
                                          kind="auto_s", gamma=gamma,
                                          reduce_dtype={A.dtype: torch.float32})
    assert _rel(res.pytree["weight"], ref.reduced[0]) < 2e-2
    exact = _exact_sq(A, G).sqrt()
    assert torch.all(scale.double() * exact <= 1.0)


def test_without_the_bound_the_estimate_under_reports(dev):
    # The hardware's own rounding on the crafted inputs: the plain estimate S
    # falls below ||G^T A||^2 by more than the bf16 guard (0.4% of the norm)
    # for some examples -- the clip factor needs the error term.
    gen = _gen(97)
    B, T, din, dout = 32, 128, 4096, 4096
    A, G = _cancelling(B, T, din, dout, 1e-3, torch.bfloat16, gen)
    sq, err = ops.gram_sqnorms(A.to(dev), G.to(dev), return_error=True)
    exact = _exact_sq(A, G)
    rel = (sq.cpu() - exact) / exact
    assert torch.all((sq.cpu() - exact).abs() <= err.cpu())
    assert (rel < -0.008).sum().item() >= 1, rel
