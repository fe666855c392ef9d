"""The allocation-free Gram-norm entry point (GPU test, through the C ABI).

``dpc_gram_sqnorms_noalloc`` takes its workspace from a static per-device
array instead of a caller's buffer.  Its squared norms and error bounds must
equal ``dpc_gram_sqnorms``'s bit for bit (the same kernels, deterministic
folds) on two calls in a row -- the second smaller, so stale records of the
first call must not leak into it -- with and without a bias and with
accumulation, for the MFMA (bf16) and generic (fp32) kernels; a call whose
workspace would exceed DPC_NOALLOC_SCRATCH_BYTES is refused with DPC_ENOSPC
before anything runs.
"""

from __future__ import annotations

import pytest
import torch

from opake_amd import _native as nat
from opake_amd import ops
from opake_amd.exceptions import OperationError

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 48 << 20


def _noalloc(A, G, *, with_bias, out=None, err=None):
    B, T, din = A.shape
    dout = G.shape[2]
    accumulate = out is not None
    if out is None:
        out = torch.empty(B, dtype=torch.float64, device=A.device)
        err = torch.empty(B, dtype=torch.float64, device=A.device)
    nat.call("dpc_gram_sqnorms_noalloc", nat.ptr(A), nat.ptr(G), B, T, din, dout,
             nat.dtype_code(A.dtype), int(with_bias), int(accumulate), nat.ptr(out), nat.ptr(err),
             nat.stream_handle(A.device))
    return out, err


def _inputs(dev, B, T, din, dout, dtype, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    A = torch.randn(B, T, din, generator=g, device=dev).to(dtype)
    G = (torch.randn(B, T, dout, generator=g, device=dev) * 0.01).to(dtype)
    return A, G


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("with_bias", [False, True])
def test_noalloc_equals_workspace_entry_point(dev, dtype, with_bias):
    # The headline shape (B = 32, T = 512: split Gram kernel, its accumulator
    # exchange in the scratch), then smaller calls.
    shapes = [(32, 512, 512, 384), (8, 512, 256, 384), (3, 130, 64, 40)]
    for k, (B, T, din, dout) in enumerate(shapes):
        assert nat.load().dpc_gram_workspace_bytes(B, T) <= SCRATCH_BYTES
        A, G = _inputs(dev, B, T, din, dout, dtype, seed=10 * k + with_bias)
        want_sq, want_err = ops.gram_sqnorms(A, G, with_bias=with_bias, return_error=True)
        got_sq, got_err = _noalloc(A, G, with_bias=with_bias)
        assert torch.equal(got_sq, want_sq), (k, B, T)
        assert torch.equal(got_err, want_err), (k, B, T)
        # Accumulating a second layer into the same vectors.
        A2, G2 = _inputs(dev, B, T, din // 2, dout, dtype, seed=10 * k + 5)
        ops.gram_sqnorms(A2, G2, with_bias=with_bias, out=want_sq, err=want_err)
        _noalloc(A2, G2, with_bias=with_bias, out=got_sq, err=got_err)
        assert torch.equal(got_sq, want_sq), (k, "accumulate")
        assert torch.equal(got_err, want_err), (k, "accumulate")


def test_noalloc_refuses_calls_beyond_its_scratch(dev):
    B, T = 64, 4096  # 64 x 2080 tile records of 96 bytes plus the split exchange: > 48 MiB
    assert nat.load().dpc_gram_workspace_bytes(B, T) > SCRATCH_BYTES
    A, G = _inputs(dev, B, T, 64, 64, torch.bfloat16, seed=1)
    with pytest.raises(OperationError, match="DPC_ENOSPC"):
        _noalloc(A, G, with_bias=False)
    # A call within the limit still works afterwards.
    A, G = _inputs(dev, 2, 256, 64, 64, torch.bfloat16, seed=2)
    sq, err = _noalloc(A, G, with_bias=False)
    want_sq, want_err = ops.gram_sqnorms(A, G, return_error=True)
    assert torch.equal(sq, want_sq) and torch.equal(err, want_err)
