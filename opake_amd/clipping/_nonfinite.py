"""Examples whose linear-layer operands hold NaN / Inf, with the reference's
semantics.

The reference materialises each per-example gradient and replaces its
non-finite entries by zero before the norm and the scale
(``nan_to_num``, packages/opake-engine/src/opake/api/engine/clipping/
_streaming.py:73,151; _pytree.py:606-613).  For a linear layer the entry
``(m, k)`` of ``G_i^T A_i`` is non-finite exactly when column ``k`` of ``A_i``
or column ``m`` of ``G_i`` holds a non-finite value (any token), so the
sanitised gradient is ``G_i'^T A_i'`` with those columns zeroed over all
tokens (``dpc_sanitize_columns``).

The ghost paths never form per-example gradients: an example with a
non-finite operand gets a non-finite Gram norm, scale 0, and is left out of
the clipped sums.  The clip-factor kernels also count those examples into a
pinned host word (``nonfinite``, written with system scope).  The host reads
the count once the norm pass has completed -- by then the clipped-sum
launches are already queued, so the GPU does not wait -- and, only when it is
not zero, clips the flagged examples the reference's way: sanitised operands,
per-example gradients from the clipped-sum kernel (scale 1, in the parameter
dtype, as ``vmap(grad)`` stores them), then the materialised-leaf kernels
with the same bounds and groups; their sums are added to the result and their
norms, scales and counts replace the flagged entries of the diagnostics.
Under HIP-graph capture the count cannot be read; flagged examples then stay
out of the sums (scale 0).
"""

from __future__ import annotations

import time

import torch

from opake_amd import ops
from opake_amd.exceptions import OperationError

MODES = ("sanitize", "drop")
_POLL_S = 0.05  # spin on the pinned word this long before a stream sync


def check_mode(mode: str) -> None:
    if mode not in MODES:
        from opake_amd.exceptions import ConfigurationError

        raise ConfigurationError(f"nonfinite must be one of {MODES}, got {mode!r}")


class NonfiniteWatch:
    """Pinned host words that clip-factor launches fill with their count of
    examples whose norm is not finite (-1 until written)."""

    def __init__(self, device: torch.device, n: int):
        self.device = device
        self.flags = torch.full((n,), -1, dtype=torch.int32, pin_memory=True)

    def slot(self, k: int) -> torch.Tensor:
        return self.flags[k:k + 1]

    def count(self) -> int:
        """Blocks until every slot is written (the norm passes completed)."""
        view = self.flags.numpy()
        deadline = time.perf_counter() + _POLL_S
        while view.min() < 0:
            if time.perf_counter() > deadline:
                torch.cuda.current_stream(self.device).synchronize()
                if view.min() < 0:
                    raise OperationError("a clip-factor pass did not report its non-finite count")
                break
        return int(view.sum())


def watch(device: torch.device, n: int, mode: str) -> NonfiniteWatch | None:
    """A watch for ``n`` clip-factor launches, or ``None`` (``drop``, or under
    graph capture, where the host cannot read a count)."""
    check_mode(mode)
    if mode == "drop" or torch.cuda.is_current_stream_capturing():
        return None
    return NonfiniteWatch(device, n)


def bad_examples(*sq_err) -> torch.Tensor:
    """Indices (int64, device) of the examples whose squared norms or bounds
    (float64 [..., B] tensors) are not finite anywhere."""
    bad = None
    for t in sq_err:
        if t is None:
            continue
        b = ~torch.isfinite(t)
        b = b.reshape(-1, b.shape[-1]).any(dim=0)
        bad = b if bad is None else bad | b
    return bad.nonzero().flatten()


def sanitized_linear_grads(A: torch.Tensor, G: torch.Tensor, dtype: torch.dtype,
                           bias: bool) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Per-example gradients of a linear layer from operands [n, T, d] with
    their non-finite columns zeroed: weight [n, dout, din] and bias [n, dout]
    (or None) in ``dtype``."""
    n = A.shape[0]
    As = ops.sanitize_columns(A)
    Gs = ops.sanitize_columns(G)
    one = torch.ones(1, dtype=torch.float32, device=A.device)
    ws = [ops.clipped_sum(As[j:j + 1], Gs[j:j + 1], one, out_dtype=dtype)[0] for j in range(n)]
    w = torch.stack(ws) if ws else torch.empty((0, G.shape[2], A.shape[2]), dtype=dtype,
                                               device=A.device)
    b = Gs.float().sum(dim=1).to(dtype) if bias else None
    return w, b


__all__ = ["MODES", "NonfiniteWatch", "bad_examples", "check_mode", "sanitized_linear_grads",
           "watch"]
