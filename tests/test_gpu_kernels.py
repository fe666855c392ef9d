"""Parity of each HIP kernel with the CPU oracle (GPU tests, called through the C ABI)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from opake_amd import _native as nat
from opake_amd import ops
from opake_amd.clipping import _numerics as num
from oracle import c_oracle, clip_oracle, ghost_oracle

pytestmark = pytest.mark.gpu

RANDOM123_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# --- Philox stream ---------------------------------------------------------


@pytest.mark.parametrize("ctr,key,expected", RANDOM123_KAT)
def test_philox_known_answers(dev, ctr, key, expected):
    got = ops.philox4x32_10(ctr, key, 1, dev).cpu().numpy()[0]
    assert tuple(int(x) for x in got) == expected


def test_philox_matches_c_oracle(dev):
    got = ops.philox4x32_10((7, 1, 2, 3), (0xDEADBEEF, 0x12345678), 4096, dev).cpu().numpy()
    want = c_oracle.philox((7, 1, 2, 3), (0xDEADBEEF, 0x12345678), 4096)
    assert np.array_equal(got.astype(np.uint32), want)


# --- squared norms -----------------------------------------------------------


def _exact_sqnorms(A, G, bias=False):
    w = torch.einsum("btm,btn->bmn", G.double(), A.double())
    sq = (w * w).sum(dim=(1, 2))
    if bias:
        sq = sq + (G.double().sum(dim=1) ** 2).sum(dim=1)
    return sq


@pytest.mark.parametrize(
    "B,T,din,dout",
    [(3, 128, 64, 64), (2, 200, 136, 72), (2, 512, 256, 128), (1, 1, 8, 8), (4, 130, 64, 40),
     # din == dout and an even number of 128-row blocks: one operand per work
     # item (diagonal and off-diagonal tile sets, a ragged last block, 16 sets)
     (2, 256, 64, 64), (3, 512, 128, 128), (2, 200, 72, 72), (2, 1024, 64, 64),
     # din == dout with an odd number of blocks: the paired kernel
     (2, 384, 96, 96)],
)
@pytest.mark.parametrize("bias", [False, True])
def test_gram_sqnorms_bf16(dev, B, T, din, dout, bias):
    g = _gen(B * 1000 + T)
    A = torch.randn(B, T, din, generator=g).to(torch.bfloat16)
    G = torch.randn(B, T, dout, generator=g).to(torch.bfloat16)
    got = ops.gram_sqnorms(A.to(dev), G.to(dev), with_bias=bias).cpu()
    want = _exact_sqnorms(A, G, bias)
    # fp32 MFMA accumulation of exact bf16 products, fp64 combination.
    torch.testing.assert_close(got, want, rtol=1e-4, atol=0)


@pytest.mark.parametrize("B,T,din,dout", [(3, 17, 33, 9), (2, 70, 64, 65)])
def test_gram_sqnorms_fp32_generic(dev, B, T, din, dout):
    g = _gen(7)
    A = torch.randn(B, T, din, generator=g)
    G = torch.randn(B, T, dout, generator=g)
    got = ops.gram_sqnorms(A.to(dev), G.to(dev), with_bias=True).cpu()
    torch.testing.assert_close(got, _exact_sqnorms(A, G, True), rtol=1e-5, atol=0)


def test_gram_sqnorms_accumulate(dev):
    g = _gen(3)
    A1, G1 = torch.randn(2, 64, 32, generator=g), torch.randn(2, 64, 16, generator=g)
    A2, G2 = torch.randn(2, 64, 24, generator=g), torch.randn(2, 64, 8, generator=g)
    out = ops.gram_sqnorms(A1.to(dev), G1.to(dev))
    ops.gram_sqnorms(A2.to(dev), G2.to(dev), out=out, return_error=False)
    torch.testing.assert_close(out.cpu(), _exact_sqnorms(A1, G1) + _exact_sqnorms(A2, G2),
                               rtol=1e-5, atol=0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_flat_sqnorms(dev, dtype):
    g = _gen(5)
    a = torch.randn(6, 784, generator=g).to(dtype)
    gg = torch.randn(6, 512, generator=g).to(dtype)
    got = ops.flat_sqnorms(a.to(dev), gg.to(dev), with_bias=True).cpu()
    want = (a.double() ** 2).sum(1) * (gg.double() ** 2).sum(1) + (gg.double() ** 2).sum(1)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=0)


def test_gram_nonfinite_example_is_nonfinite(dev):
    g = _gen(9)
    A = torch.randn(3, 128, 64, generator=g).to(torch.bfloat16)
    G = torch.randn(3, 128, 64, generator=g).to(torch.bfloat16)
    A[1, 5, 7] = float("nan")
    G[2, 3, 1] = float("inf")
    got = ops.gram_sqnorms(A.to(dev), G.to(dev)).cpu()
    assert math.isfinite(got[0].item())
    assert not math.isfinite(got[1].item())
    assert not math.isfinite(got[2].item())


# --- clip factors ---------------------------------------------------------------


def _oracle_scales(sq, C, rel_abs_storage, kind="fixed", gamma=0.0, err=None):
    storage, mult, roundoff = rel_abs_storage
    up = sq if err is None else sq + err
    up = torch.where(up < 0, torch.zeros_like(up), up)  # NaN stays NaN
    norm = torch.sqrt(up)
    bound = torch.clamp(torch.as_tensor(C, dtype=torch.float64), min=0.0)
    ratio = bound / (norm + gamma) if kind == "auto_s" else bound / norm
    return clip_oracle.finalize_scale(ratio, storage, mult, roundoff, clamp_to_one=kind != "auto_s")


@pytest.mark.parametrize("kind", ["fixed", "auto_s"])
@pytest.mark.parametrize("with_err", [False, True])
def test_clip_factors_bit_exact(dev, kind, with_err):
    g = _gen(11)
    B = 3000
    sq = torch.exp(torch.randn(B, generator=g, dtype=torch.float64) * 3)
    sq[:6] = torch.tensor([0.0, math.inf, math.nan, 1.0, 0.25, 1e300], dtype=torch.float64)
    err = None
    if with_err:
        # An error bound per example (a cancelled estimate may even be
        # negative: the scale then comes from the bound alone).
        err = sq * torch.rand(B, generator=g, dtype=torch.float64) * 0.01
        err[3] = 0.5
        sq[8], err[8] = -0.125, 1.0
    # Scales 2^-65 .. 2^-75 (positive in float32, below the plan's 2^-64
    # fast-list bound) in each of the kernel's 1024-example passes.
    for i, e in ((7, 130), (1500, 140), (2047, 150), (2999, 134)):
        sq[i] = 2.0 ** e
    C = clip_oracle.conservative_bound(1.0)
    gamma = 0.01 if kind == "auto_s" else 0.0
    guards = []
    expect = []
    for storage in (torch.bfloat16, torch.float32):
        mult = torch.promote_types(storage, torch.float32)
        roundoff = clip_oracle.norm_roundoff(torch.float32, torch.float64, 1, 10240)
        guards.append(num.guard_constants(storage, mult, roundoff))
        expect.append(_oracle_scales(sq, C, (storage, mult, roundoff), kind, gamma,
                                     err).to(torch.float32))
    cf = ops.clip_factors(sq.to(dev), C, guards, err=None if err is None else err.to(dev),
                          kind=nat.SCALE_AUTO_S if kind == "auto_s" else nat.SCALE_FIXED,
                          gamma=gamma, count_threshold=1.0)
    for gi in range(2):
        assert torch.equal(cf.scale[gi].cpu(), expect[gi]), gi
    norms = torch.sqrt(torch.where(sq < 0, torch.zeros_like(sq), sq)).to(torch.float32)
    torch.testing.assert_close(cf.norms.cpu(), norms, rtol=0, atol=0, equal_nan=True)
    assert int(cf.nclipped.item()) == int((norms > 1.0).sum().item())
    # Plan: examples with a positive guard-0 scale; those at or above 2^-64
    # from the front in increasing order, the others from the back (B * C is
    # far below the 2^55 bound here).
    # One plan per guard: the examples with a positive scale; those in
    # [2^-64, 2^32] from the front in increasing order, the others from the
    # back (B * C is far below the 2^55 bound here).
    for gi in range(2):
        s0 = expect[gi]
        fast = [i for i in range(B) if 2.0 ** -64 <= s0[i] <= 2.0 ** 32]
        slow = [i for i in range(B) if 0 < s0[i] and not 2.0 ** -64 <= s0[i] <= 2.0 ** 32]
        assert slow == [7, 1500, 2047, 2999]
        plan = cf.plan[gi].cpu().numpy().view(np.int32)
        assert plan[0] == len(fast) + len(slow)
        assert plan[1] == len(fast)
        active = plan[4:4 + B]
        assert list(active[:len(fast)]) == fast
        assert list(active[B - len(slow):][::-1]) == slow


def _plan_lists(plan, B):
    """Per guard: (nactive, nfast, front list, back list) -- the words a plan
    defines (the rest of its buffer is never written)."""
    out = []
    for p in plan.cpu().numpy():
        w = p.view(np.int32)
        nact, nfast = int(w[0]), int(w[1])
        act = w[4:4 + B]
        out.append((nact, nfast, act[:nfast].tolist(), act[B - (nact - nfast):].tolist()))
    return out


@pytest.mark.parametrize("G,B", [(8, 300), (70, 37)])
def test_clip_factors_groups_match_per_group_calls(dev, G, B):
    """One launch over G groups equals G dpc_clip_factors calls bit for bit
    (scales, float64 scales, norms, counts, plans, non-finite counts), groups
    past the 64 of one launch included."""
    g = _gen(23)
    sq = torch.exp(torch.randn(G, B, generator=g, dtype=torch.float64) * 3)
    err = sq * torch.rand(G, B, generator=g, dtype=torch.float64) * 0.01
    sq[0, :3] = torch.tensor([math.nan, math.inf, 0.0], dtype=torch.float64)
    sq[G - 1, 5] = 2.0 ** 140  # a slow-list example
    err[1, 4] = math.nan
    Cs = [0.5 + 0.25 * k for k in range(G)]
    thr = [float(np.float32(c)) for c in Cs]
    roundoff = clip_oracle.norm_roundoff(torch.float32, torch.float64, 2, 4096)
    guards = [(*num.guard_constants(torch.bfloat16, torch.float32, roundoff), True),
              (*num.guard_constants(torch.float64, torch.float64, roundoff), torch.float64)]
    sq_d, err_d = sq.to(dev), err.to(dev)
    nf = torch.full((G,), -1, dtype=torch.int32, device=dev)
    got = ops.clip_factors_groups(sq_d, Cs, guards, err=err_d, count_thresholds=thr,
                                  nonfinite=nf)
    for k in range(G):
        nf1 = torch.full((1,), -1, dtype=torch.int32, device=dev)
        want = ops.clip_factors(sq_d[k], Cs[k], guards, err=err_d[k], count_threshold=thr[k],
                                nonfinite=nf1)
        one = got.group(k)
        assert torch.equal(one.scale.cpu(), want.scale.cpu()), k
        assert torch.equal(one.scale64.cpu(), want.scale64.cpu()), k
        torch.testing.assert_close(one.norms.cpu(), want.norms.cpu(), rtol=0, atol=0,
                                   equal_nan=True)
        assert torch.equal(one.nclipped.cpu(), want.nclipped.cpu()), k
        assert _plan_lists(one.plan, B) == _plan_lists(want.plan, B), k
        assert int(nf[k]) == int(nf1[0]), k
    assert int(nf[0]) == 2 and int(nf[1]) == 1


@pytest.mark.parametrize("accumulate", [0, 1])
def test_group_sum_column_major_and_accumulate(dev, accumulate):
    """dpc_group_sum_f64 over a column-major [B, n] block: per-group sums in
    column order from 0.0, added to the output when accumulating -- the same
    fp64 additions as a sequential host loop."""
    g = _gen(29)
    B, n, G = 45, 13, 4
    x = torch.randn(n, B, generator=g, dtype=torch.float64)  # column j is row j
    groups = [int(v) for v in torch.randint(0, G, (n,), generator=g)]
    base = torch.randn(G, B, generator=g, dtype=torch.float64)
    out = base.clone().to(dev)
    col_group = torch.tensor(groups, dtype=torch.int32, device=dev)
    xd = x.to(dev)
    nat.call("dpc_group_sum_f64", nat.ptr(xd), B, n, 1, B, nat.ptr(col_group), G,
             nat.ptr(out), accumulate, nat.stream_handle(torch.device(dev)))
    want = torch.empty(G, B, dtype=torch.float64)
    for gg in range(G):
        for b in range(B):
            s = 0.0
            for j in range(n):
                if groups[j] == gg:
                    s += float(x[j, b])
            want[gg, b] = base[gg, b] + s if accumulate else s
    assert torch.equal(out.cpu(), want)
    # A layout where neither dimension steps over the other is refused.
    rc = nat.load().dpc_group_sum_f64(nat.ptr(xd), B, n, 2, 2, nat.ptr(col_group), G,
                                      nat.ptr(out), 0, nat.stream_handle(torch.device(dev)))
    assert rc == nat.DPC_EINVAL


def test_clip_factors_boundary_example(dev):
    # The reference's own boundary pin: [[3,4],[0.6,0.8]], C=1 -> [1.2, 1.6]
    # (an example at ||g|| == C is still scaled by rel < 1).
    sq = torch.tensor([25.0, 1.0], dtype=torch.float64)
    roundoff = clip_oracle.norm_roundoff(torch.float32, torch.float64, 1, 2)
    guard = num.guard_constants(torch.float32, torch.float32, roundoff)
    cf = ops.clip_factors(sq.to(dev), 1.0, [guard], count_threshold=1.0)
    s = cf.scale[0].cpu().double()
    vals = torch.tensor([[3.0, 4.0], [0.6, 0.8]], dtype=torch.float32)
    out = (vals * s.float().view(2, 1)).sum(0)
    torch.testing.assert_close(out, torch.tensor([1.2, 1.6]))
    assert s[1] < 1.0
    assert int(cf.nclipped.item()) == 1


# --- clipped sum -----------------------------------------------------------------


def _oracle_clipped_sum(A, G, C, nb=1.0, bias=False, out_dtype=None, kind="fixed", gamma=0.0):
    leaves = ghost_oracle.linear_per_example_grads(A, G, with_bias=bias)
    red = {A.dtype: out_dtype} if out_dtype is not None else None
    res = clip_oracle.stream_clip_and_sum(leaves, clip_oracle.conservative_bound(C), kind=kind,
                                          gamma=gamma, reduce_dtype=red)
    return [clip_oracle.normalize(r, nb) for r in res.reduced], res


def _run_clipped_sum(dev, A, G, C, nb=1.0, bias=False, out_dtype=None, use_plan=True):
    B, T, din = A.shape
    dout = G.shape[2]
    sq, err = ops.gram_sqnorms(A.to(dev), G.to(dev), with_bias=bias, return_error=True) \
        if T > 1 else ops.flat_sqnorms(A[:, 0].to(dev), G[:, 0].to(dev), with_bias=bias,
                                       return_error=True)
    from opake_amd.clipping import guard_for_linear
    cf = ops.clip_factors(sq, num.conservative_bound(C), [guard_for_linear(A.dtype, din, dout, bias)],
                          err=err, count_threshold=num.float32_of(C))
    w, b = ops.clipped_sum(A.to(dev), G.to(dev), cf.scale[0], plan=cf.plan[0] if use_plan else None,
                           normalize_by=nb, out_dtype=out_dtype, with_bias=bias)
    return w, b, cf


def _rel_err(got, want):
    got, want = got.double(), want.double()
    return ((got - want).norm() / want.norm().clamp_min(1e-300)).item()


@pytest.mark.parametrize(
    "B,T,din,dout",
    [(4, 128, 256, 256), (3, 64, 320, 264), (5, 192, 512, 136), (2, 64, 8, 8)],
)
def test_clipped_sum_bf16_mfma(dev, B, T, din, dout):
    g = _gen(B + T + din)
    A = torch.randn(B, T, din, generator=g).to(torch.bfloat16)
    G = (torch.randn(B, T, dout, generator=g) * 0.01 *
         torch.exp(torch.randn(B, 1, 1, generator=g))).to(torch.bfloat16)
    w, _, cf = _run_clipped_sum(dev, A, G, 1.0, nb=float(B), out_dtype=torch.float32)
    (want,), res = _oracle_clipped_sum(A, G, 1.0, nb=float(B), out_dtype=torch.float32)
    assert _rel_err(w.cpu(), want) < 2e-2
    torch.testing.assert_close(cf.norms.cpu().double(), res.norms, rtol=2e-2, atol=0)


def test_clipped_sum_accumulator_scaling_is_near_exact(dev):
    """The bf16 GEMM applies each example's scale to its fp32 accumulators
    (no bf16 rounding of the scaled operand): against the exact clipped sum in
    float64 the error is far below the bf16-rounding level (2^-9)."""
    B, T, din, dout = 6, 128, 256, 256
    g = _gen(77)
    A = torch.randn(B, T, din, generator=g).to(torch.bfloat16)
    G = (torch.randn(B, T, dout, generator=g) * 0.01 *
         torch.exp(torch.randn(B, 1, 1, generator=g))).to(torch.bfloat16)
    w, _, cf = _run_clipped_sum(dev, A, G, 1.0, out_dtype=torch.float32)
    scale = cf.scale[0].cpu().double()
    exact = torch.einsum("b,btm,btn->mn", scale, G.double(), A.double())
    assert _rel_err(w.cpu(), exact) < 1e-5


# Several layers' Gram norms in one call (dpc_gram_sqnorms_multi): the sums
# (and error bounds) equal consecutive accumulating gram_sqnorms calls bit
# for bit -- one shared split launch (bf16, an even number of 128-row
# blocks, B % 8 == 0; layers of different widths, run longest first and
# summed in the caller's order) and the layer-by-layer fallbacks (B = 6,
# T = 300, 9 layers); with and without sums already in out / err.
@pytest.mark.parametrize("B,T,n,acc", [(8, 256, 3, False), (16, 512, 5, True), (6, 256, 3, False),
                                       (8, 300, 2, True), (8, 256, 9, False)])
def test_gram_sqnorms_multi_matches_consecutive_calls(dev, B, T, n, acc):
    g = _gen(B * 100 + T + n)
    dims = [(256, 264), (512, 128), (64, 1024), (1024, 64), (136, 8), (8, 520), (320, 320),
            (96, 200), (48, 56)][:n]
    As = [torch.randn(B, T, din, generator=g).to(torch.bfloat16).to(dev) for din, _ in dims]
    Gs = [(torch.randn(B, T, dout, generator=g) * torch.exp(torch.randn(B, 1, 1, generator=g)))
          .to(torch.bfloat16).to(dev) for _, dout in dims]
    start = torch.rand(B, generator=g, dtype=torch.float64).to(dev) if acc else None
    want = start.clone() if acc else None
    want_err = start.clone() * 1e-6 if acc else None
    for i, (a, x) in enumerate(zip(As, Gs)):
        if i == 0 and not acc:
            want, want_err = ops.gram_sqnorms(a, x, return_error=True)
        else:
            ops.gram_sqnorms(a, x, out=want, err=want_err)
    out = start.clone() if acc else None
    err = start.clone() * 1e-6 if acc else None
    if acc:
        got, got_err = ops.gram_sqnorms_multi(As, Gs, out=out, err=err)
    else:
        got, got_err = ops.gram_sqnorms_multi(As, Gs, return_error=True)
    assert torch.equal(got, want)
    assert torch.equal(got_err, want_err)
    # And the sums are the layers' norms: against float64 on the host.
    if not acc:
        ref = sum(ghost_oracle.linear_per_example_grads(a.cpu(), x.cpu(), dtype=torch.float64)[0]
                  .pow(2).sum(dim=(1, 2)) for a, x in zip(As, Gs))
        torch.testing.assert_close(got.cpu(), ref, rtol=1e-4, atol=0)


def _multi_case(dev, dims, B, T, seed, slow=False):
    g = _gen(seed)
    As = [torch.randn(B, T, din, generator=g).to(torch.bfloat16) for din, _ in dims]
    Gs = []
    for _, dout in dims:
        G = torch.randn(B, T, dout, generator=g) * 0.01 * torch.exp(torch.randn(B, 1, 1, generator=g))
        if slow:
            # Example 1's norm ~6e20 (scale below 2^-64: the plan's slow
            # slots) with its Gram entries (~5e36) still finite in fp32.
            G[1] = torch.randn(T, dout, generator=g) * 1e17
        Gs.append(G.to(torch.bfloat16))
    As_d, Gs_d = [a.to(dev) for a in As], [x.to(dev) for x in Gs]
    sq = torch.zeros(B, dtype=torch.float64, device=dev)
    err = torch.zeros(B, dtype=torch.float64, device=dev)
    for a, x in zip(As_d, Gs_d):
        ops.gram_sqnorms(a, x, out=sq, err=err)
    from opake_amd.clipping import guard_for_linear
    guard = guard_for_linear(torch.bfloat16, max(d for d, _ in dims), max(o for _, o in dims), False)
    cf = ops.clip_factors(sq, num.conservative_bound(1.0), [guard], err=err,
                          count_threshold=num.float32_of(1.0))
    return As, Gs, As_d, Gs_d, cf


# Layers of one clipping group in shared launches (dpc_clipped_sum_multi):
# mixed shapes -- one output tile (8 x 8), partial tiles (264, 136, 520
# rows), several tiles -- and 11 layers (two launches of up to 8).  Each
# layer equals its own one-layer launch bit for bit (float32 output; bfloat16
# with / normalize_by and Philox noise, whose values depend only on the
# layer's leaf id), and the exact float64 clipped sum with the device's
# scales to 1e-5; with an example on the plan's slow slots the oracle's
# clipped sum to 2e-2 (its G is scaled and rounded to bf16 first).
@pytest.mark.parametrize("case", ["mixed", "eleven", "noise_bf16", "slow"])
def test_clipped_sum_multi_matches_single_layers(dev, case):
    B, T = 3, 128
    if case == "eleven":
        dims = [(64 + 32 * i, 8 + 64 * (i % 4)) for i in range(11)]
    else:
        dims = [(256, 264), (320, 136), (64, 520), (512, 256), (8, 8)]
    As, Gs, As_d, Gs_d, cf = _multi_case(dev, dims, B, T, 100 + len(case), slow=case == "slow")
    nplan = cf.plan[0].cpu().view(torch.int32)
    assert int(nplan[1]) == (B - 1 if case == "slow" else B)  # fast examples
    kw = dict(plan=cf.plan[0], out_dtype=torch.float32)
    noises = None
    if case == "noise_bf16":
        kw = dict(plan=cf.plan[0], out_dtype=torch.bfloat16, normalize_by=2.0)
        noises = [ops.NoiseSpec(sigma=0.5 + 0.1 * i, mode=nat.NOISE_PHILOX, seed=77, leaf_id=3 * i)
                  for i in range(len(dims))]
        noises[1] = None  # a layer without noise among noisy ones
    got = ops.clipped_sum_multi(As_d, Gs_d, cf.scale[0], noises=noises, **kw)
    for i in range(len(dims)):
        one = ops.clipped_sum_multi([As_d[i]], [Gs_d[i]], cf.scale[0],
                                    noises=None if noises is None else [noises[i]], **kw)[0]
        assert got[i].shape == (dims[i][1], dims[i][0])
        assert torch.equal(got[i], one), i
    scale = cf.scale[0].cpu().double()
    for i in range(len(dims)):
        if case == "noise_bf16":
            break
        if case == "slow":
            leaves = [ghost_oracle.linear_per_example_grads(a, x)[0] for a, x in zip(As, Gs)]
            res = clip_oracle.stream_clip_and_sum(leaves, clip_oracle.conservative_bound(1.0),
                                                  reduce_dtype={torch.bfloat16: torch.float32})
            assert _rel_err(got[i].cpu(), res.reduced[i]) < 2e-2, i
        else:
            exact = torch.einsum("b,btm,btn->mn", scale, Gs[i].double(), As[i].double())
            assert _rel_err(got[i].cpu(), exact) < 1e-5, i


@pytest.mark.parametrize("case", ["tiny_scale", "large_bc"])
def test_clipped_sum_slow_plan_slots(dev, case):
    """Examples the GEMM cannot divide its accumulators by -- a scale below
    2^-64 (gradient norm ~3e20 here, Gram entries still finite in fp32), or
    every example when B * C > 2^55 --
    take the slow slots of the clip plan (G scaled before the product); the
    result matches the oracle, and the fast examples around them are intact."""
    B, T, din, dout = 5, 128, 256, 264
    g = _gen(91)
    A = torch.randn(B, T, din, generator=g).to(torch.bfloat16)
    G = torch.randn(B, T, dout, generator=g) * 0.01
    C = 1.0
    if case == "tiny_scale":
        G[2] *= 1e19  # norm ~3e20: scale ~3e-21 < 2^-64
    else:
        C = 1e17  # B * C > 2^55: no example is clipped, all take the slow slots
    G = G.to(torch.bfloat16)
    w, _, cf = _run_clipped_sum(dev, A, G, C, out_dtype=torch.float32)
    plan = cf.plan[0].cpu().view(torch.int32)
    nactive, nfast = int(plan[0]), int(plan[1])
    assert nactive == B
    assert nfast == (B - 1 if case == "tiny_scale" else 0)
    (want,), res = _oracle_clipped_sum(A, G, C, out_dtype=torch.float32)
    assert _rel_err(w.cpu(), want) < 2e-2
    torch.testing.assert_close(cf.norms.cpu().double(), res.norms, rtol=2e-2, atol=0)


def test_clipped_sum_ignores_the_plan_gap(dev):
    """A plan with fast, slow and zero-scale examples leaves entries between
    its two lists unwritten (the buffer is not cleared).  The GEMM reads
    neither them nor the scales they would index: with the gap filled with an
    out-of-range index the sum still matches the fp64 reference built from
    the device's scales."""
    B, T, din, dout = 6, 128, 256, 264
    g = _gen(93)
    A = torch.randn(B, T, din, generator=g).to(torch.bfloat16)
    G = (torch.randn(B, T, dout, generator=g) * 0.01).to(torch.bfloat16)
    A_d, G_d = A.to(dev), G.to(dev)
    sq, err = ops.gram_sqnorms(A_d, G_d, return_error=True)
    sq[1] = 1e42  # scale ~1e-21 < 2^-64: the slow list
    sq[3] = float("nan")  # scale 0: in neither list
    from opake_amd.clipping import guard_for_linear
    cf = ops.clip_factors(sq, num.conservative_bound(1.0),
                          [guard_for_linear(A.dtype, din, dout, False)], err=err,
                          count_threshold=num.float32_of(1.0))
    plan = cf.plan[0].view(torch.int32)
    nactive, nfast = int(plan[0]), int(plan[1])
    assert (nactive, nfast) == (B - 1, B - 2)
    nslow = nactive - nfast
    plan[4 + nfast:4 + B - nslow] = 0x7FFFFFFF  # the gap: one entry here
    torch.cuda.synchronize()
    w, _ = ops.clipped_sum(A_d, G_d, cf.scale[0], plan=cf.plan[0], out_dtype=torch.float32)
    s = cf.scale[0].cpu().double()
    assert s[3] == 0 and 0 < s[1] < 2.0 ** -64
    want = torch.einsum("b,btm,btk->mk", s, G.double(), A.double())
    assert _rel_err(w.cpu(), want) < 2e-2


@pytest.mark.parametrize("B,T,din,dout", [(8, 256, 512, 264), (16, 128, 256, 256)])
def test_clipped_sum_split_k(dev, B, T, din, dout):
    """Launches of few output tiles split their K steps (2-8 slices through the
    workspace, added in a fixed order): same result as the oracle, the same
    bits on every run, and the fused Philox noise equal to the noise kernel's."""
    # The workspace holds at least two fp32 K slices of the output.
    assert nat.load().dpc_clipped_sum_workspace_bytes(B, T, din, dout, nat.DPC_BF16) >= \
        2 * din * dout * 4
    g = _gen(B * T + din)
    A = torch.randn(B, T, din, generator=g).to(torch.bfloat16)
    G = (torch.randn(B, T, dout, generator=g) * 0.01 *
         torch.exp(torch.randn(B, 1, 1, generator=g))).to(torch.bfloat16)
    w, b, cf = _run_clipped_sum(dev, A, G, 1.0, nb=2.0, bias=True, out_dtype=torch.float32)
    (wb, ww), _ = _oracle_clipped_sum(A, G, 1.0, nb=2.0, bias=True, out_dtype=torch.float32)
    assert _rel_err(w.cpu(), ww) < 2e-2
    assert _rel_err(b.cpu(), wb) < 2e-2
    w2, _, _ = _run_clipped_sum(dev, A, G, 1.0, nb=2.0, bias=True, out_dtype=torch.float32)
    assert torch.equal(w, w2)
    kw = dict(plan=cf.plan[0], normalize_by=2.0, out_dtype=torch.bfloat16)
    center, _ = ops.clipped_sum(A.to(dev), G.to(dev), cf.scale[0], **kw)
    spec = ops.NoiseSpec(sigma=0.5, mode=nat.NOISE_PHILOX, seed=7, leaf_id=3)
    noisy, _ = ops.clipped_sum(A.to(dev), G.to(dev), cf.scale[0], noise=spec, **kw)
    assert torch.equal(noisy, ops.add_noise(center, 0.5, mode=nat.NOISE_PHILOX, seed=7, leaf_id=3))


def test_clipped_sum_bf16_out_and_bias(dev):
    g = _gen(21)
    A = torch.randn(3, 128, 256, generator=g).to(torch.bfloat16)
    G = (torch.randn(3, 128, 128, generator=g) * 0.02).to(torch.bfloat16)
    w, b, _ = _run_clipped_sum(dev, A, G, 0.5, nb=2.0, bias=True)
    (wb, ww), _ = _oracle_clipped_sum(A, G, 0.5, nb=2.0, bias=True)
    assert w.dtype == torch.bfloat16 and b.dtype == torch.bfloat16
    assert _rel_err(w.cpu(), ww) < 2e-2
    assert _rel_err(b.cpu(), wb) < 2e-2


# The last three split K over 4-6 workgroups per tile (fp32 partials added in a
# fixed order by the reduce kernel, which applies the epilogue): the config-1
# layers at B = 256 / 300 and a ragged K with an empty last slice.
@pytest.mark.parametrize("B,T,din,dout", [(6, 1, 784, 512), (3, 5, 33, 17), (4, 3, 64, 10),
                                          (256, 1, 784, 512), (300, 1, 512, 10),
                                          (130, 3, 96, 34)])
def test_clipped_sum_fp32_generic(dev, B, T, din, dout):
    g = _gen(31)
    A = torch.randn(B, T, din, generator=g)
    G = torch.randn(B, T, dout, generator=g) * 0.05
    w, b, cf = _run_clipped_sum(dev, A, G, 1.0, nb=float(B), bias=True)
    (wb, ww), res = _oracle_clipped_sum(A, G, 1.0, nb=float(B), bias=True)
    torch.testing.assert_close(cf.norms.cpu().double(), res.norms, rtol=1e-5, atol=0)
    assert _rel_err(w.cpu(), ww) < 1e-5
    assert _rel_err(b.cpu(), wb) < 1e-5
    w2, _, _ = _run_clipped_sum(dev, A, G, 1.0, nb=float(B), bias=True)
    assert torch.equal(w, w2)


# bf16 at T = 64: the MFMA kernel's clip plan; fp32 at T = 1: the generic
# kernel's one-token path (16 examples per chunk, each row scaled by its own
# example's scale), whose zero-scale rows must not be read either.
@pytest.mark.parametrize("dtype,B,T,tol", [(torch.bfloat16, 3, 64, 2e-2),
                                           (torch.float32, 40, 1, 1e-5)])
def test_clipped_sum_plan_skips_nonfinite_examples(dev, dtype, B, T, tol):
    g = _gen(41)
    A = torch.randn(B, T, 64, generator=g).to(dtype)
    G = (torch.randn(B, T, 64, generator=g) * 0.01).to(dtype)
    A[1, 0, 0] = float("nan")
    if B > 3:
        G[17, 0, 3] = float("inf")
    w, _, cf = _run_clipped_sum(dev, A, G, 1.0, out_dtype=torch.float32)
    assert torch.isfinite(w).all()
    assert cf.scale[0, 1].item() == 0.0
    keep = torch.tensor([i for i in range(B) if i not in (1, 17)])
    assert all(cf.scale[0, i].item() > 0.0 for i in keep.tolist())
    (want,), _ = _oracle_clipped_sum(A[keep], G[keep], 1.0, out_dtype=torch.float32)
    assert _rel_err(w.cpu(), want) < tol


def test_clipped_sum_fast_and_generic_agree(dev):
    g = _gen(51)
    A = torch.randn(4, 128, 256, generator=g).to(torch.bfloat16)
    G = (torch.randn(4, 128, 256, generator=g) * 0.01).to(torch.bfloat16)
    w_fast, _, _ = _run_clipped_sum(dev, A, G, 1.0, out_dtype=torch.float32, use_plan=True)
    w_gen, _, _ = _run_clipped_sum(dev, A, G, 1.0, out_dtype=torch.float32, use_plan=False)
    assert _rel_err(w_fast.cpu(), w_gen.cpu()) < 5e-3


# --- noise ---------------------------------------------------------------------


# Shapes on both launch layouts: a flat thread index (narrow leaves) and one
# row pair per workgroup row (columns a multiple of 256, or at least 2048).
@pytest.mark.parametrize("shape", [(37, 19), (5, 512), (3, 2100)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_add_noise_injected_bit_exact(dev, dtype, shape):
    from oracle import noise_oracle

    g = _gen(61)
    x = torch.randn(*shape, generator=g).to(dtype)
    z = torch.randn(*shape, generator=g)
    y = ops.add_noise(x.to(dev), 0.7, mode=nat.NOISE_INJECTED, noise=z.to(dev)).cpu()
    assert torch.equal(y, noise_oracle.sample(x, 0.7, z))


# The grouped noise gives every leaf exactly add_noise's values: 37 leaves
# (two launches of up to 32), flat and row-block shapes, a 1-D leaf, an empty
# one, a scalar, sigma 0 (copied, -0.0 kept), out of place and in place.
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("inplace", [False, True])
def test_add_noise_leaves_matches_per_leaf(dev, dtype, inplace):
    g = _gen(71)
    shapes = [(64, 33), (7,), (5, 3, 4), (7, 768), (3, 2100), (0, 5), (), (16, 4096)]
    shapes = (shapes * 5)[:37]
    xs = [torch.randn(sh, generator=g).to(dtype).to(dev) for sh in shapes]
    xs[2].view(-1)[0] = -0.0
    sigmas = [0.0 if i % 7 == 2 else 0.25 + 0.1 * i for i in range(len(xs))]
    ids = [3 * i + 1 for i in range(len(xs))]
    seed = 0x0F1E2D3C4B5A6978
    want = [ops.add_noise(x, s, mode=nat.NOISE_PHILOX, seed=seed, leaf_id=i)
            for x, s, i in zip(xs, sigmas, ids)]
    ins = [x.clone() for x in xs]
    got = ops.add_noise_leaves(ins, sigmas, seed=seed, leaf_ids=ids, inplace=inplace)
    bits = torch.int16 if dtype == torch.bfloat16 else torch.int32
    for k, (a, b) in enumerate(zip(got, want)):
        assert a.shape == b.shape, k
        assert torch.equal(a.view(bits), b.view(bits)), k
        if a.numel():
            assert (a.data_ptr() == ins[k].data_ptr()) == inplace, k
    assert torch.equal(got[2].reshape(-1)[:1].view(bits), xs[2].reshape(-1)[:1].view(bits))


@pytest.mark.parametrize("shape", [(64, 33), (7,), (5, 3, 4), (7, 768), (3, 2100), (2, 4, 1024),
                                   (3, 2049)])
def test_add_noise_device_stream_matches_c_oracle(dev, shape):
    x = torch.zeros(shape)
    seed = 0x0123456789ABCDEF
    y = ops.add_noise(x.to(dev), 1.0, mode=nat.NOISE_PHILOX, seed=seed, leaf_id=3).cpu()
    rows, cols = ops.leaf_view(x)
    want = torch.from_numpy(c_oracle.leaf_normals(seed, 3, rows, cols)).reshape(shape)
    # The device evaluates the transform in float (normals within 1e-6 of the
    # double-precision formulas).
    torch.testing.assert_close(y.double(), want, rtol=0, atol=5e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_add_noise_misaligned_leaf_matches_aligned(dev, dtype):
    # A leaf starting one element into its storage is not 8-byte aligned and
    # takes the one-column kernel; the aligned copy takes the two-column one.
    g = _gen(67)
    flat = torch.randn(1 + 5 * 1024, generator=g).to(dtype).to(dev)
    x = flat[1:].view(5, 1024)
    assert x.data_ptr() % 8 != 0
    seed = 0x5EED
    y = ops.add_noise(x, 0.5, mode=nat.NOISE_PHILOX, seed=seed, leaf_id=2)
    y_aligned = ops.add_noise(x.clone(), 0.5, mode=nat.NOISE_PHILOX, seed=seed, leaf_id=2)
    assert torch.equal(y.cpu(), y_aligned.cpu())
    z = torch.randn(5, 1024, generator=g)
    zf = torch.zeros(1 + z.numel())
    zf[1:] = z.flatten()
    zv = zf.to(dev)[1:].view(5, 1024)
    yi = ops.add_noise(x, 0.5, mode=nat.NOISE_INJECTED, noise=zv)
    yi_aligned = ops.add_noise(x.clone(), 0.5, mode=nat.NOISE_INJECTED, noise=z.to(dev))
    assert torch.equal(yi.cpu(), yi_aligned.cpu())


def test_clipped_sum_epilogue_noise_injected_bit_exact(dev):
    from oracle import noise_oracle

    g = _gen(71)
    A = torch.randn(2, 64, 256, generator=g).to(torch.bfloat16)
    G = (torch.randn(2, 64, 256, generator=g) * 0.01).to(torch.bfloat16)
    sq = ops.gram_sqnorms(A.to(dev), G.to(dev))
    from opake_amd.clipping import guard_for_linear
    cf = ops.clip_factors(sq, 1.0, [guard_for_linear(torch.bfloat16, 256, 256, False)],
                          count_threshold=1.0)
    for out_dtype in (torch.float32, torch.bfloat16):
        center, _ = ops.clipped_sum(A.to(dev), G.to(dev), cf.scale[0], plan=cf.plan[0],
                                    normalize_by=4.0, out_dtype=out_dtype)
        z = torch.randn(256, 256, generator=g)
        noisy, _ = ops.clipped_sum(
            A.to(dev), G.to(dev), cf.scale[0], plan=cf.plan[0], normalize_by=4.0, out_dtype=out_dtype,
            noise=ops.NoiseSpec(sigma=0.25, mode=nat.NOISE_INJECTED, noise=z.to(dev)))
        assert torch.equal(noisy.cpu(), noise_oracle.sample(center.cpu(), 0.25, z))


def test_clipped_sum_epilogue_noise_philox_matches_add_noise(dev):
    g = _gen(81)
    A = torch.randn(2, 64, 264, generator=g).to(torch.bfloat16)
    G = (torch.randn(2, 64, 136, generator=g) * 0.01).to(torch.bfloat16)
    sq = ops.gram_sqnorms(A.to(dev), G.to(dev))
    from opake_amd.clipping import guard_for_linear
    cf = ops.clip_factors(sq, 1.0, [guard_for_linear(torch.bfloat16, 264, 136, True)],
                          count_threshold=1.0)
    kw = dict(plan=cf.plan[0], normalize_by=2.0, out_dtype=torch.float32, with_bias=True)
    cw, cb = ops.clipped_sum(A.to(dev), G.to(dev), cf.scale[0], **kw)
    spec = ops.NoiseSpec(sigma=0.5, mode=nat.NOISE_PHILOX, seed=99, leaf_id=1, bias_leaf_id=0)
    nw, nbias = ops.clipped_sum(A.to(dev), G.to(dev), cf.scale[0], noise=spec, **kw)
    ew = ops.add_noise(cw, 0.5, mode=nat.NOISE_PHILOX, seed=99, leaf_id=1)
    eb = ops.add_noise(cb, 0.5, mode=nat.NOISE_PHILOX, seed=99, leaf_id=0)
    assert torch.equal(nw, ew)
    assert torch.equal(nbias, eb)


def test_timing_event_measures_a_launch(dev):
    """The fence-free timing events (dpc_timing_event_*) bracket work on the
    current stream like torch's: a 64 MiB copy, timed by both, agrees to
    within a factor of 2 and is positive."""
    x = torch.empty(16 << 20, device=dev)
    y = torch.empty_like(x)
    y.copy_(x)
    a, b = nat.TimingEvent(), nat.TimingEvent()
    ta, tb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ta.record()
    a.record()
    for _ in range(10):
        y.copy_(x)
    b.record()
    tb.record()
    torch.cuda.synchronize()
    ms, ms_torch = a.elapsed_time(b), ta.elapsed_time(tb)
    assert ms > 0.0
    assert 0.5 * ms_torch < ms <= ms_torch * 1.01 + 0.05
