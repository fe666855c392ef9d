"""Host-side closed forms of the clipping guard.

These are scalar computations on dtype metadata (``torch.finfo``) that
configure the kernels; no tensor data passes through here.  They restate
``packages/opake-engine/src/opake/api/engine/clipping/_pytree.py``:

* ``compute_dtype_for_reduction`` - ``_resolve_compute_dtype_for_reduction``
  (:84-108);
* ``guard_constants`` - the ``relative`` / ``absolute`` of ``_guard_scale``
  (:111-141), which the clip-factor kernel applies as ``ratio * rel - abs``;
* ``reduction_terms`` / ``norm_roundoff`` - ``_reduction_terms`` (:252-268) and
  ``_norm_roundoff`` (:271-283) for a leaf set given by per-example sizes;
* ``conservative_bound`` - ``_conservative_bound_tensor``
  (``_clipped_fun.py:206-216``): C as float32, one ulp down if rounding went up.
"""

from __future__ import annotations

import math

import torch

REDUCTION_BLOCK = 2048
BLOCKED_REDUCTION_MIN = 4096


def _real(dtype: torch.dtype) -> torch.dtype:
    if not dtype.is_complex:
        return dtype
    return {torch.complex64: torch.float32, torch.complex128: torch.float64}[dtype]


def compute_dtype_for_reduction(leaf_dtypes, compute_dtype=None) -> torch.dtype:
    if compute_dtype is not None:
        return compute_dtype
    acc = torch.float32
    for dt in leaf_dtypes:
        if not (dt.is_floating_point or dt.is_complex):
            continue
        r = _real(dt)
        acc = torch.promote_types(acc, torch.float32 if r in (torch.float16, torch.bfloat16) else r)
    return acc


def guard_constants(storage: torch.dtype, multiply: torch.dtype, roundoff: float):
    s = torch.finfo(_real(storage))
    m = torch.finfo(_real(multiply))
    rounding = s.eps if multiply == storage else s.eps / 2.0 + m.eps
    return 1.0 - rounding - 2.0 * roundoff, s.smallest_normal * s.eps


def reduction_terms(numels) -> int:
    widest = max([0, *numels])
    if widest <= 1:
        return 0
    if widest > BLOCKED_REDUCTION_MIN:
        return REDUCTION_BLOCK + (widest + REDUCTION_BLOCK - 1) // REDUCTION_BLOCK
    return widest


def norm_roundoff(acc: torch.dtype, sq: torch.dtype, n_leaves: int, n_reduction: int) -> float:
    u_acc = torch.finfo(acc).eps / 2.0
    u_sq = torch.finfo(sq).eps / 2.0
    return (u_acc + (max(n_leaves, 1) + n_reduction) * u_sq) / 2.0


def conservative_bound(value: float) -> float:
    exact = float(value)
    bound = torch.tensor(exact, dtype=torch.float32)
    if bound.item() > exact:
        bound = torch.nextafter(bound, torch.tensor(-math.inf, dtype=torch.float32))
    return float(bound.item())


def float32_of(value: float) -> float:
    """``value`` rounded to float32 (nearest), as a Python float."""
    return float(torch.tensor(float(value), dtype=torch.float32).item())


__all__ = [
    "compute_dtype_for_reduction",
    "conservative_bound",
    "float32_of",
    "guard_constants",
    "norm_roundoff",
    "reduction_terms",
]
