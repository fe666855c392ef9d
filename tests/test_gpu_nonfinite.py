"""NaN / Inf in the operands of the ghost paths, against the materialised
oracle (GPU tests).

The reference zeroes the non-finite entries of each per-example gradient and
clips the rest (packages/opake-engine/src/opake/api/engine/clipping/
_streaming.py:73,151; _pytree.py:606-613; test
packages/opake-engine/tests/clipping/test_clipped_grad.py:65-83).  The
oracle does exactly that on per-example gradients materialised in float64
and rounded to the parameter dtype (``ghost_oracle.linear_per_example_grads``
/ ``segment_grads``) followed by ``stream_clip_and_sum``.  Planted: a lone
NaN in one activation, a whole token row of Inf in the output gradients, an
example whose activations are all NaN, and a NaN in one output-gradient
column -- beside finite examples -- on the dense bf16 path (split Gram
kernel and the one-launch norm + clip), the generic float32 path, a flat
(T = 1) layer, and the grouped (mixture-of-experts) path.

Tolerances: bf16 inputs 2e-2 relative (``north_star``: the Gram norm of
the exact product vs the norm of its bf16-rounded copy), float32 1e-5; the
flagged examples' norms, computed from the same rounded per-example
gradients as the oracle's, 1e-3.
"""

from __future__ import annotations

import math

import pytest
import torch

from opake_amd.clipping import LinearCapture, ghost_clip_captured, ghost_clip_sum
from opake_amd.types import PerGroup
from oracle import clip_oracle, ghost_oracle

pytestmark = pytest.mark.gpu


def _rel(got, want):
    got, want = got.double().cpu(), want.double().cpu()
    return ((got - want).norm() / want.norm().clamp_min(1e-300)).item()


def _plant(A, G):
    """Examples 1-4 get non-finite values; 0 and 5.. stay finite."""
    A, G = A.clone(), G.clone()
    A[1, 3, 5] = math.nan                  # a lone NaN in one activation
    G[2, 7, :] = math.inf                  # a whole token row of Inf
    A[3] = math.nan                        # every activation NaN
    G[4, :, 2] = -math.inf                 # one output-gradient column
    return A, G


def _inputs(B, T, din, dout, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    A = torch.randn(B, T, din, generator=gen)
    scale = torch.exp(torch.randn(B, 1, 1, generator=gen))
    G = torch.randn(B, T, dout, generator=gen) * scale / math.sqrt(T * din * dout)
    return _plant(A.to(dtype), G.to(dtype))


@pytest.mark.parametrize("dtype,T,din,dout,bias", [
    (torch.bfloat16, 256, 128, 128, False),   # split Gram kernel, norms + clip in one launch
    (torch.bfloat16, 130, 64, 96, True),      # MFMA Gram with a bias, generic GEMM (T % 64)
    (torch.float32, 96, 40, 24, False),       # generic fp32 kernels
    (torch.float32, 1, 40, 24, True),         # flat (T = 1) norms
])
@pytest.mark.parametrize("auto_s", [None, 0.01])
def test_ghost_clip_sum_nonfinite_matches_oracle(dev, dtype, T, din, dout, bias, auto_s):
    B = 7
    if T == 1:
        # One token: a "row" of Inf is the example's whole output gradient.
        A, G = _inputs(B, 8, din, dout, dtype, seed=T + din)
        A, G = A[:, :1].contiguous(), G[:, :1].contiguous()
        A[1, 0, 5] = math.nan
        G[4, 0, 2] = math.inf
    else:
        A, G = _inputs(B, T, din, dout, dtype, seed=T + din)
    C = 0.8
    res, aux = ghost_clip_sum(A.to(dev), G.to(dev), clipping_norm=C, bias=bias, return_aux=True,
                              auto_s_gamma=auto_s, dtype=torch.float32)
    leaves = ghost_oracle.linear_per_example_grads(A, G, with_bias=bias)
    want = clip_oracle.stream_clip_and_sum(leaves, clip_oracle.conservative_bound(C),
                                           kind="auto_s" if auto_s else "fixed",
                                           gamma=auto_s or 0.0)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    names = ["bias", "weight"] if bias else ["weight"]
    for n, w in zip(names, want.reduced):
        got = res.pytree[n]
        assert torch.isfinite(got).all(), n
        assert _rel(got, w) < tol, n
    norms = aux.grad_norms.cpu().double()
    assert torch.isfinite(norms).all()
    torch.testing.assert_close(norms, want.norms, rtol=tol, atol=1e-30)
    # All-NaN activations: every weight-gradient entry is zeroed (the bias
    # gradient, from the finite output gradients, survives).
    if T > 1 and not bias:
        assert norms[3].item() == 0.0
    # The DP bound holds for every example, the flagged ones included.
    assert torch.all(aux.clipped_grad_norms.cpu().double() <= C * (1 + 1e-6))
    if auto_s is None and dtype == torch.float32:
        assert int(aux.num_clipped.item()) == int((want.norms.float() > C).sum())


def test_ghost_clip_sum_nonfinite_drop_mode(dev):
    # nonfinite="drop": the flagged examples get scale 0 and no contribution.
    A, G = _inputs(6, 256, 128, 128, torch.bfloat16, seed=3)
    res, aux = ghost_clip_sum(A.to(dev), G.to(dev), clipping_norm=0.8, return_aux=True,
                              dtype=torch.float32, nonfinite="drop")
    scales = aux.clip_scales.cpu()
    assert torch.all(scales[1:5] == 0.0) and torch.all(scales[[0, 5]] > 0.0)
    keep = [0, 5]
    leaves = ghost_oracle.linear_per_example_grads(A[keep], G[keep])
    want = clip_oracle.stream_clip_and_sum(leaves, clip_oracle.conservative_bound(0.8))
    assert _rel(res.pytree["weight"], want.reduced[0]) < 2e-2


@pytest.mark.parametrize("per_group", [False, True])
def test_ghost_clip_captured_nonfinite_grouped(dev, per_group):
    """A dense layer and two row-segmented (expert) layers: an Inf in the dense
    layer's output gradient and a NaN in expert 0's rows of example 2, an
    all-NaN expert-1 segment of example 3."""
    gen = torch.Generator().manual_seed(11)
    B, T, d, h = 5, 64, 64, 128
    A = torch.randn(B, T, d, generator=gen).to(torch.bfloat16)
    G = (torch.randn(B, T, h, generator=gen) * 0.01).to(torch.bfloat16)
    segs = [[20, 0, 37, 12, 5], [11, 30, 0, 19, 41]]
    experts = []
    for e, lens in enumerate(segs):
        rows = sum(lens)
        a = torch.randn(rows, h, generator=gen).to(torch.bfloat16)
        g = (torch.randn(rows, d, generator=gen) * 0.02).to(torch.bfloat16)
        experts.append((a, g, lens))
    G[2, 9, 17] = math.inf                           # dense layer, example 2
    experts[0][0][20 + 0 + 3, 4] = math.nan          # expert 0, a row of example 2
    start3 = sum(segs[1][:3])
    experts[1][0][start3:start3 + segs[1][3]] = math.nan  # expert 1, example 3: all NaN
    caps = [LinearCapture(name="dense", A=A.to(dev), G=G.to(dev))]
    for e, (a, g, lens) in enumerate(experts):
        caps.append(LinearCapture(name=f"experts.{e}", A=a.to(dev), G=g.to(dev), segments=lens))
    if per_group:
        norm = PerGroup({"dense.weight": "d", "experts.0.weight": "e", "experts.1.weight": "e"},
                        {"d": 0.5, "e": 0.7})
    else:
        norm = 0.6
    res, aux = ghost_clip_captured(caps, clipping_norm=norm, return_aux=True, dtype=torch.float32)
    leaves = {"dense.weight": ghost_oracle.linear_per_example_grads(A, G)[0]}
    for e, (a, g, lens) in enumerate(experts):
        leaves[f"experts.{e}.weight"] = ghost_oracle.segment_grads(a, g, lens,
                                                                    dtype=torch.bfloat16)
    names = sorted(leaves)
    if per_group:
        assignment = {"dense.weight": "d", "experts.0.weight": "e", "experts.1.weight": "e"}
        values = {k: clip_oracle.conservative_bound(v) for k, v in norm.values.items()}
        want = clip_oracle.stream_clip_and_sum([leaves[n] for n in names], None,
                                               groups=[assignment[n] for n in names],
                                               group_values=values)
    else:
        want = clip_oracle.stream_clip_and_sum([leaves[n] for n in names],
                                               clip_oracle.conservative_bound(norm))
    for n, w in zip(names, want.reduced):
        got = res.pytree[n]
        assert torch.isfinite(got).all(), n
        assert _rel(got, w) < 2e-2, n
    if per_group:
        for g in ("d", "e"):
            torch.testing.assert_close(aux.group_norms[g].cpu().double(), want.group_norms[g],
                                       rtol=2e-2, atol=1e-30)
    else:
        torch.testing.assert_close(aux.grad_norms.cpu().double(), want.norms, rtol=2e-2,
                                   atol=1e-30)
