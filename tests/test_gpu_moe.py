"""GPU parity of the grouped (row-segmented) path: mixture-of-experts layers.

Kernel level: ``grouped_gram_sqnorms`` and ``grouped_clipped_sum`` against the
materialised per-segment gradients of the oracle (``segment_grads``) on ragged
segments -- empty ones, lengths that are not multiples of the 64-row step or
the 128-row Gram tile, and a segment holding NaN whose scale is 0.  Model
level: ``ghost_clipped_grad`` on a ``TopKMoE`` against per-example gradients
computed by a loop of single-example backward passes, clipped per expert by the
streaming oracle.  Tolerances: 1e-5 relative for float32, 2e-2 relative for
bfloat16 inputs with float32 accumulation.
"""

from __future__ import annotations

import math

import pytest
import torch

from opake_amd import _native as nat
from opake_amd import ops
from opake_amd.clipping import auto_ghost_clipped_grad, ghost_clipped_grad
from opake_amd.moe import TopKMoE, expert_groups
from opake_amd.noise import gaussian_noise
from opake_amd.random import key
from opake_amd.types import NoisedPytree, PerGroup
from oracle import clip_oracle, ghost_oracle

pytestmark = pytest.mark.gpu


def _rel(got, want):
    got, want = got.double().cpu(), want.double().cpu()
    return ((got - want).norm() / want.norm().clamp_min(1e-300)).item()


def _problem(gen, lengths, din, dout, dtype, nan_segment=None):
    As, Gs = [], []
    for e, lens in enumerate(lengths):
        rows = sum(lens)
        A = torch.randn(rows, din, generator=gen)
        G = torch.randn(rows, dout, generator=gen) * 0.05
        if nan_segment is not None and nan_segment[0] == e:
            k = nan_segment[1]
            r0 = sum(lens[:k])
            A[r0, 0] = math.nan
            G[r0 + lens[k] - 1, 1] = math.inf
        As.append(A.to(dtype))
        Gs.append(G.to(dtype))
    return As, Gs


LENGTHS = [[0, 1, 63, 64, 65], [130, 0, 200, 7, 128], [256, 300, 2, 0, 64]]


@pytest.mark.parametrize("dtype,din,dout", [(torch.float32, 40, 24), (torch.bfloat16, 64, 96),
                                            (torch.bfloat16, 36, 20)])
def test_grouped_gram_sqnorms_match_segment_grads(dev, dtype, din, dout):
    gen = torch.Generator().manual_seed(din)
    As, Gs = _problem(gen, LENGTHS, din, dout, dtype)
    layout = ops.SegmentLayout(LENGTHS, dev)
    got = ops.grouped_gram_sqnorms([a.to(dev) for a in As], [g.to(dev) for g in Gs], layout)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for e, lens in enumerate(LENGTHS):
        want = ghost_oracle.segment_grads(As[e], Gs[e], lens, dtype=torch.float64)
        sq = (want ** 2).sum(dim=(1, 2))
        for k in range(len(lens)):
            if lens[k] == 0:
                assert got[e, k].item() == 0.0
            else:
                assert abs(got[e, k].item() - sq[k].item()) <= tol * sq[k].item(), (e, k)


@pytest.mark.parametrize("dtype,shapes", [
    (torch.bfloat16, [(64, 96), (128, 40), (32, 256)]),
    (torch.bfloat16, [(64, 96), (36, 40), (32, 256)]),  # one misaligned width: generic kernel
    (torch.float32, [(24, 16), (40, 8), (8, 48)]),
])
def test_grouped_gram_mixed_shapes_cost_ordered(dev, dtype, shapes):
    gen = torch.Generator().manual_seed(17)
    As, Gs = [], []
    for lens, (din, dout) in zip(LENGTHS, shapes):
        rows = sum(lens)
        As.append(torch.randn(rows, din, generator=gen).to(dtype))
        Gs.append((torch.randn(rows, dout, generator=gen) * 0.1).to(dtype))
    layout = ops.SegmentLayout(LENGTHS, dev, gram_weights=[a + b for a, b in shapes])
    got = ops.grouped_gram_sqnorms([a.to(dev) for a in As], [g.to(dev) for g in Gs], layout)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for e, lens in enumerate(LENGTHS):
        want = (ghost_oracle.segment_grads(As[e], Gs[e], lens, dtype=torch.float64) ** 2).sum(
            dim=(1, 2))
        for k in range(len(lens)):
            assert abs(got[e, k].item() - want[k].item()) <= tol * want[k].item(), (e, k)


# Segments for the grouped split kernel (1 .. 320 rows: up to 8 units of 32
# rows, a ninth (257 .. 288) and a tenth (289 .. 320)) beside longer ones
# that take the tile-pair kernel in the same call.
SPLIT_LENGTHS = [[1, 31, 32, 33, 127, 128, 129, 200, 255, 256],
                 [257, 270, 287, 288, 289, 0, 64, 96, 160, 321],
                 [250, 260, 280, 300, 8, 16, 319, 320, 190, 240]]


def _all_pairs_sqnorms(dev, As, Gs, layout):
    """The same call with every segment on the tile-pair kernel."""
    import ctypes

    dims = (ctypes.c_int * (2 * layout.E))(
        *[v for A, G in zip(As, Gs) for v in (A.shape[1], G.shape[1])])
    sq = torch.empty((layout.E, layout.K), dtype=torch.float64, device=dev)
    err = torch.empty_like(sq)
    nbytes = nat.load().dpc_grouped_gram_workspace_bytes(layout.n_items, 0)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    a_ptrs = torch.tensor([a.data_ptr() for a in As], dtype=torch.int64, device=dev)
    g_ptrs = torch.tensor([g.data_ptr() for g in Gs], dtype=torch.int64, device=dev)
    nat.call("dpc_grouped_gram_sqnorms", nat.ptr(a_ptrs), nat.ptr(g_ptrs), dims, layout.E,
             nat.DPC_BF16, nat.ptr(layout.items), layout.n_launch_items, layout.max_rows,
             nat.ptr(None), 0, 0, layout.n_items, nat.ptr(layout.item_start), layout.S,
             nat.ptr(sq), nat.ptr(err), nat.ptr(ws), ws.numel(), nat.stream_handle(dev))
    return sq, err


@pytest.mark.parametrize("dims", [[(64, 96), (128, 40), (32, 256)],
                                  [(256, 256), (96, 160), (512, 64)]])
def test_grouped_split_kernel_matches_exact(dev, dims):
    """The grouped split kernel's segment norms: within their own error bound
    of the exact fp64 ||G_v^T A_v||^2 (so the clip factor is DP-sound), and
    within 2e-2 of it; the tile-pair kernel on the same segments agrees."""
    gen = torch.Generator().manual_seed(sum(a for a, _ in dims))
    As, Gs = [], []
    for lens, (din, dout) in zip(SPLIT_LENGTHS, dims):
        rows = sum(lens)
        scale = torch.exp(torch.randn(rows, 1, generator=gen))
        As.append(torch.randn(rows, din, generator=gen).to(torch.bfloat16))
        Gs.append((torch.randn(rows, dout, generator=gen) * 0.1 * scale).to(torch.bfloat16))
    layout = ops.SegmentLayout(SPLIT_LENGTHS, dev, gram_dims=dims)
    assert layout.n_set_items > 0 and layout.n_long_items > 0
    Ad, Gd = [a.to(dev) for a in As], [g.to(dev) for g in Gs]
    for rep in range(2):  # the tickets are cleared for every call
        sq, err = ops.grouped_gram_sqnorms(Ad, Gd, layout, return_error=True)
        sq, err = sq.cpu(), err.cpu()
        for e, lens in enumerate(SPLIT_LENGTHS):
            exact = (ghost_oracle.segment_grads(As[e], Gs[e], lens, dtype=torch.float64) ** 2
                     ).sum(dim=(1, 2))
            for k, n in enumerate(lens):
                if n == 0:
                    assert sq[e, k].item() == 0.0 and err[e, k].item() == 0.0
                    continue
                d = abs(sq[e, k].item() - exact[k].item())
                assert d <= err[e, k].item(), (rep, e, k, n, d, err[e, k].item())
                assert d <= 2e-2 * exact[k].item(), (rep, e, k, n)
                assert err[e, k].item() <= 1e-2 * exact[k].item(), (rep, e, k, n)
    psq, perr = _all_pairs_sqnorms(dev, Ad, Gd, layout)
    torch.testing.assert_close(sq, psq.cpu(), rtol=1e-5, atol=0)


@pytest.mark.parametrize("dtype,din,dout", [(torch.float32, 40, 24), (torch.bfloat16, 264, 136),
                                            (torch.bfloat16, 36, 20)])
@pytest.mark.parametrize("out_dtype", [None, torch.float32])
def test_grouped_clipped_sum_matches_segment_grads(dev, dtype, din, dout, out_dtype):
    gen = torch.Generator().manual_seed(din + dout)
    As, Gs = _problem(gen, LENGTHS, din, dout, dtype, nan_segment=(1, 2))
    layout = ops.SegmentLayout(LENGTHS, dev)
    scale = torch.rand(len(LENGTHS), len(LENGTHS[0]), generator=gen)
    scale[0, 3] = 0.0
    scale[1, 2] = 0.0  # the segment with NaN / Inf is never read
    out = ops.grouped_clipped_sum([a.to(dev) for a in As], [g.to(dev) for g in Gs], layout,
                                  scale.to(dev), normalize_by=3.0, out_dtype=out_dtype)
    assert out.dtype == (out_dtype or dtype)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for e, lens in enumerate(LENGTHS):
        grads = ghost_oracle.segment_grads(As[e], Gs[e], lens, dtype=torch.float64)
        want = sum(scale[e, k].double() * grads[k] for k in range(len(lens)) if scale[e, k] > 0)
        assert torch.isfinite(out[e].float()).all()
        assert _rel(out[e], want / 3.0) < tol, e


def test_grouped_fast_and_generic_agree(dev):
    # din = 264 takes the MFMA kernel; din = 260 (not a multiple of 8) the generic one.
    gen = torch.Generator().manual_seed(9)
    As, Gs = _problem(gen, LENGTHS, 264, 64, torch.bfloat16)
    layout = ops.SegmentLayout(LENGTHS, dev)
    scale = torch.rand(3, 5, generator=gen).to(dev)
    fast = ops.grouped_clipped_sum([a.to(dev) for a in As], [g.to(dev) for g in Gs], layout, scale,
                                   out_dtype=torch.float32)
    cut = [a[:, :260].contiguous().to(dev) for a in As]
    slow = ops.grouped_clipped_sum(cut, [g.to(dev) for g in Gs], layout, scale,
                                   out_dtype=torch.float32)
    assert _rel(fast[:, :, :260], slow) < 1e-2


@pytest.mark.parametrize("mode", ["philox", "injected"])
def test_grouped_epilogue_noise_matches_add_noise(dev, mode):
    gen = torch.Generator().manual_seed(2)
    As, Gs = _problem(gen, LENGTHS, 64, 128, torch.bfloat16)
    layout = ops.SegmentLayout(LENGTHS, dev)
    scale = torch.rand(3, 5, generator=gen).to(dev)
    args = ([a.to(dev) for a in As], [g.to(dev) for g in Gs], layout, scale)
    sigmas = [0.5, 0.0, 2.0]
    clean = ops.grouped_clipped_sum(*args, normalize_by=2.0, out_dtype=torch.float32)
    if mode == "philox":
        spec = ops.GroupedNoise(sigmas=sigmas, mode=nat.NOISE_PHILOX, seed=1234,
                                leaf_ids=[7, 3, 11])
    else:
        draws = [torch.randn(128, 64, generator=gen).to(dev) for _ in range(3)]
        spec = ops.GroupedNoise(sigmas=sigmas, mode=nat.NOISE_INJECTED, noise=draws)
    noisy = ops.grouped_clipped_sum(*args, normalize_by=2.0, out_dtype=torch.float32, noise=spec)
    for e in range(3):
        if mode == "philox":
            want = ops.add_noise(clean[e], sigmas[e], mode=nat.NOISE_PHILOX, seed=1234,
                                 leaf_id=[7, 3, 11][e])
        else:
            want = ops.add_noise(clean[e], sigmas[e], mode=nat.NOISE_INJECTED, noise=draws[e])
        assert torch.equal(noisy[e], want), e


# --- model level -------------------------------------------------------------------


def _mse(out, t):
    return ((out.float() - t.float()) ** 2).sum(dim=(1, 2))


def _moe_case(dtype, d, inter, E, B, T, seed=0):
    torch.manual_seed(seed)
    model = TopKMoE(d, inter, E, 2, dtype=torch.float32)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0.0, 0.02 * math.sqrt(64.0 / d))
    gen = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(B, T, d, generator=gen)
    logits = torch.randn(B, T, E, generator=gen)
    target = torch.randn(B, T, d, generator=gen)
    ref_model = model.double() if dtype == torch.float32 else model.to(dtype).double()
    return ref_model, x, logits, target


def _oracle(model, x, logits, target, clipping_norm, names, kind="fixed", gamma=0.0):
    per = ghost_oracle.per_example_grads_loop(model, _mse, (x.double(), logits.double()),
                                              target.double())
    leaves = [per[n].float() for n in names]
    if isinstance(clipping_norm, PerGroup):
        groups = [clipping_norm.groups[(n,)] for n in names]
        values = {g: clip_oracle.conservative_bound(v) for g, v in clipping_norm.values.items()}
        return clip_oracle.stream_clip_and_sum(leaves, None, groups=groups, group_values=values,
                                               kind=kind, gamma=gamma)
    return clip_oracle.stream_clip_and_sum(leaves, clip_oracle.conservative_bound(clipping_norm),
                                           kind=kind, gamma=gamma)


@pytest.mark.parametrize("per_group", [True, False])
def test_ghost_moe_float32_matches_per_example_oracle(dev, per_group):
    ref, x, logits, target = _moe_case(torch.float32, 48, 40, 4, 4, 50)
    model = TopKMoE(48, 40, 4, 2).to(dev)
    model.load_state_dict({k: v.float() for k, v in ref.state_dict().items()})
    C = expert_groups(model, clipping_norm=0.5) if per_group else 0.5
    names = sorted(n for n, p in model.named_parameters() if p.requires_grad)
    res = _oracle(ref, x, logits, target, C, names)
    fn, st = ghost_clipped_grad(model, _mse, clipping_norm=C, normalize_by=4.0, return_aux=True)
    (out, aux), _ = fn((x.to(dev), logits.to(dev)), target.to(dev), state=st)
    assert sorted(out.pytree) == names
    for i, n in enumerate(names):
        assert _rel(out.pytree[n], res.reduced[i] / 4.0) < 1e-5, n
    if per_group:
        for gname in sorted(C.values):
            torch.testing.assert_close(aux.group_norms[gname].cpu().double(),
                                       res.group_norms[gname], rtol=1e-5, atol=0)
        assert aux.clipping_rate is None
    else:
        torch.testing.assert_close(aux.grad_norms.cpu().double(), res.norms, rtol=1e-5, atol=0)


@pytest.mark.parametrize("per_group", [True, False])
def test_ghost_moe_auto_s_matches_per_example_oracle(dev, per_group):
    # AUTO-S on the grouped (per-expert) path: R_k / (||g_k|| + gamma) per
    # example and group, no min(1, .), the scaled norms below R_k.
    ref, x, logits, target = _moe_case(torch.float32, 48, 40, 4, 4, 50, seed=9)
    model = TopKMoE(48, 40, 4, 2).to(dev)
    model.load_state_dict({k: v.float() for k, v in ref.state_dict().items()})
    R = expert_groups(model, clipping_norm=0.5) if per_group else 0.5
    names = sorted(n for n, p in model.named_parameters() if p.requires_grad)
    res = _oracle(ref, x, logits, target, R, names, kind="auto_s", gamma=0.01)
    fn, st = auto_ghost_clipped_grad(model, _mse, R=R, gamma=0.01, normalize_by=4.0,
                                     return_aux=True)
    (out, aux), _ = fn((x.to(dev), logits.to(dev)), target.to(dev), state=st)
    for i, n in enumerate(names):
        assert _rel(out.pytree[n], res.reduced[i] / 4.0) < 1e-5, n
    if per_group:
        for k, gname in enumerate(sorted(R.values)):
            torch.testing.assert_close(aux.group_norms[gname].cpu().double(),
                                       res.group_norms[gname], rtol=1e-5, atol=0)
            scaled = aux.clip_scales[k][0].double() * aux.group_norms[gname].double()
            assert torch.all(scaled <= R.values[gname])
    else:
        torch.testing.assert_close(aux.grad_norms.cpu().double(), res.norms, rtol=1e-5, atol=0)
        assert torch.all(aux.clipped_grad_norms.double() <= 0.5)


def test_ghost_moe_bf16_matches_per_example_oracle(dev):
    d, inter, E, B, T = 128, 192, 4, 4, 160
    ref, x, logits, target = _moe_case(torch.bfloat16, d, inter, E, B, T, seed=3)
    x = x.to(torch.bfloat16)
    model = TopKMoE(d, inter, E, 2, dtype=torch.bfloat16).to(dev)
    model.load_state_dict({k: v.to(torch.bfloat16) for k, v in ref.state_dict().items()})
    C = expert_groups(model, clipping_norm=0.05)
    names = sorted(n for n, p in model.named_parameters() if p.requires_grad)
    res = _oracle(ref, x.float(), logits, target, C, names)
    fn, st = ghost_clipped_grad(model, _mse, clipping_norm=C, return_aux=True,
                                dtype=torch.float32)
    (out, aux), _ = fn((x.to(dev), logits.to(dev)), target.to(dev), state=st)
    for i, n in enumerate(names):
        assert _rel(out.pytree[n], res.reduced[i]) < 2e-2, n
    for gname in sorted(C.values):
        assert _rel(aux.group_norms[gname], res.group_norms[gname]) < 2e-2, gname


@pytest.mark.parametrize("stream", ["reference", "device"])
def test_ghost_moe_fused_noise_equals_separate_noise(dev, stream):
    model = TopKMoE(64, 96, 4, 2, dtype=torch.bfloat16).to(dev)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0.0, 0.02)
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(3, 64, 64, generator=gen).to(torch.bfloat16).to(dev)
    logits = torch.randn(3, 64, 4, generator=gen).to(dev)
    target = torch.randn(3, 64, 64, generator=gen).to(dev)
    C = expert_groups(model, clipping_norm=1.0)
    fn, st = ghost_clipped_grad(model, _mse, clipping_norm=C, normalize_by=3.0,
                                dtype=torch.float32)
    noise_fn, nstate = gaussian_noise(noise_multiplier=1.3, key=key(5), stream=stream)
    fused, _, nstate2 = fn((x, logits), target, state=st, noise_fn=noise_fn, noise_state=nstate)
    plain, _ = fn((x, logits), target, state=st)
    separate, nstate3 = noise_fn(plain, nstate)
    assert isinstance(fused, NoisedPytree)
    assert nstate2._step_counter == nstate3._step_counter == 1
    for n in sorted(plain.pytree):
        assert torch.equal(fused.pytree[n], separate.pytree[n]), n
