"""``dpc_gram_clip_factors``: the Gram norms and the clip factors of one linear
layer in one launch (the split Gram kernel's last work item folds the
records and computes the clip factors).  Against the two-call path
(``dpc_gram_sqnorms`` then ``dpc_clip_factors``), bit for bit, on call after
call on one workspace (each call must leave its tickets zero for the next),
for fixed and AUTO-S scales, several guards, and the shapes that take the
separate launches inside the entry point (a bias, an odd number of 128-row
blocks, float32) interleaved with one-launch calls.
"""

from __future__ import annotations

import pytest
import torch

from opake_amd import _native as nat
from opake_amd import ops
from opake_amd.clipping import guard_for_linear

pytestmark = pytest.mark.gpu


def _inputs(dev, B, T, din, dout, dtype, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    A = torch.randn(B, T, din, generator=g, device=dev).to(dtype)
    scale = torch.exp(torch.randn(B, 1, 1, generator=g, device=dev))
    G = (torch.randn(B, T, dout, generator=g, device=dev) * 1e-4 * scale).to(dtype)
    return A, G


def _plans(plan, B):
    """The defined words of each guard's plan: nactive, nfast, the fast list
    (front) and the other list (back)."""
    out = []
    for g in range(plan.shape[0]):
        w = plan[g].cpu().view(torch.int32)
        nactive, nfast = int(w[0]), int(w[1])
        active = w[4:4 + B].tolist()
        out.append((nactive, nfast, active[:nfast], active[B - (nactive - nfast):]))
    return out


def _two_calls(A, G, C, guards, bias, kind, gamma):
    sq, err = ops.gram_sqnorms(A, G, with_bias=bias, return_error=True)
    cf = ops.clip_factors(sq, C, guards, err=err, kind=kind, gamma=gamma, count_threshold=C)
    return sq, err, cf


CASES = [
    # B, T, din, dout, dtype, bias: one launch, then the separate launches
    (32, 512, 512, 384, torch.bfloat16, False),
    (8, 256, 256, 256, torch.bfloat16, False),
    (4, 384, 128, 256, torch.bfloat16, False),   # odd block count: separate launches
    (6, 256, 128, 64, torch.bfloat16, True),     # bias: separate launches
    (5, 130, 72, 40, torch.float32, False),      # float32: separate launches
    (32, 512, 512, 384, torch.bfloat16, False),  # one launch again on the same workspace
    (16, 1024, 256, 512, torch.bfloat16, False),
]


@pytest.mark.parametrize("kind,gamma", [(nat.SCALE_FIXED, 0.0), (nat.SCALE_AUTO_S, 0.01)])
def test_gram_clip_factors_equals_two_calls(dev, kind, gamma):
    for k, (B, T, din, dout, dtype, bias) in enumerate(CASES):
        A, G = _inputs(dev, B, T, din, dout, dtype, seed=100 * k + kind)
        C = 1.0
        guards = [guard_for_linear(dtype, din, dout, bias)]
        if k % 2 == 0:  # a second guard with a bfloat16 multiply
            guards.append((*guards[0][:2], torch.bfloat16))
        for rep in range(2):  # twice in a row: the tickets were left zero
            sq, err, cf = ops.gram_clip_factors(A, G, C, guards, with_bias=bias, kind=kind,
                                                gamma=gamma, count_threshold=C)
            wsq, werr, wcf = _two_calls(A, G, C, guards, bias, kind, gamma)
            assert torch.equal(sq, wsq), (k, rep)
            assert torch.equal(err, werr), (k, rep)
            assert torch.equal(cf.scale, wcf.scale), (k, rep)
            assert torch.equal(cf.norms, wcf.norms), (k, rep)
            assert torch.equal(cf.nclipped, wcf.nclipped), (k, rep)
            assert _plans(cf.plan, B) == _plans(wcf.plan, B), (k, rep)


def test_gram_clip_factors_leaves_counters_zero(dev):
    # The counter buffer is zero after every call, whatever the shape.
    for B, T, din, dout in [(8, 512, 256, 256), (32, 512, 512, 384), (3, 256, 128, 64)]:
        A, G = _inputs(dev, B, T, din, dout, torch.bfloat16, seed=B)
        guards = [guard_for_linear(torch.bfloat16, din, dout, False)]
        ops.gram_clip_factors(A, G, 1.0, guards, count_threshold=1.0)
        torch.cuda.synchronize()
        counters = ops._GRAM_CLIP_COUNTERS[(str(dev), nat.stream_handle(dev).value or 0)]
        assert counters.numel() * 4 >= nat.load().dpc_gram_clip_counter_bytes(B, T)
        assert torch.count_nonzero(counters).item() == 0, (B, T)
