"""``clip_pytree`` / ``auto_scale_pytree`` for one example's pytree, on the GPU.

Same signatures, return values and edge cases as the reference
(packages/opake-engine/src/opake/api/engine/clipping/_pytree.py:379-649):

* NaN / Inf elements count as zero, in the norm and in the output;
* the scale is ``min(1, C / ||x||)`` (``clip_pytree``) or ``R / (||x|| + gamma)``
  (``auto_scale_pytree``, no ``min(1)``), shrunk by the final cast's rounding
  margin, computed against the exact bound (no float32 rounding of ``C``);
* ``C = 0`` gives zeros, ``C = inf`` passes through, a zero pytree is returned
  unchanged, ``return_zero`` zeroes the output;
* with ``PerGroup`` bounds each group is scaled by its own norm and bound and
  ``aux.group_norms`` holds the per-group norms.

The work is the batch kernels at batch size 1: a batch of one example summed
over the batch is that example's stored values, bit for bit.  Non-tensor
leaves pass through untouched.
"""

from __future__ import annotations

from collections import namedtuple
from typing import Any

import torch

from opake_amd.clipping._leaves import _group_layout, leaves_clip_sum, unsupported_reason
from opake_amd.exceptions import ConfigurationError, OperationError
from opake_amd.pytree import tree_flatten_with_paths, tree_unflatten
from opake_amd.types import PerGroup

ClipPytreeAux = namedtuple("ClipPytreeAux", ["norm", "group_norms"])


class _Kind:
    def __init__(self, kind: str, gamma: float = 0.0):
        self.kind = kind
        self.gamma = gamma


def _scale_one(pytree: Any, bound, kind: _Kind, *, return_zero: bool,
               compute_dtype) -> tuple[Any, ClipPytreeAux]:
    paths, flat, treedef = tree_flatten_with_paths(pytree)
    positions = [i for i, x in enumerate(flat) if isinstance(x, torch.Tensor)]
    leaves = [flat[i] for i in positions]
    grouped = isinstance(bound, PerGroup)
    names = None
    if grouped:
        names, leaf_groups, bounds = _group_layout([paths[i] for i in positions], bound)
    if not leaves:
        raise OperationError("clip_pytree on a pytree without tensor leaves is not supported")
    stacked = [leaf.detach().unsqueeze(0) for leaf in leaves]
    if any(leaf.requires_grad for leaf in leaves) and torch.is_grad_enabled():
        raise OperationError("HIP clip_pytree does not differentiate through the clip")
    reason = unsupported_reason(stacked, 1.0, kind, compute_dtype=compute_dtype,
                                second_moment=False, batch_size=1)
    if reason is not None:
        raise OperationError(f"HIP clip_pytree cannot serve this call: {reason}")
    # One example: its "batch sum" is the stored value itself, kept in the
    # storage dtype.
    keep = {leaf.dtype: (leaf.dtype, leaf.dtype) for leaf in leaves}
    if grouped:
        res = leaves_clip_sum(stacked, bounds, kind=kind.kind, gamma=kind.gamma,
                              leaf_groups=leaf_groups, conservative=False, sum_dtypes=keep,
                              compute_dtype=compute_dtype)
    else:
        res = leaves_clip_sum(stacked, float(bound), kind=kind.kind, gamma=kind.gamma,
                              conservative=False, sum_dtypes=keep, compute_dtype=compute_dtype)
    out = list(flat)
    for j, i in enumerate(positions):
        out[i] = torch.zeros_like(leaves[j]) if return_zero else res.reduced[j]
    group_norms = None
    if grouped:
        group_norms = {n: res.group_norms[k, 0] for k, n in enumerate(names)}
    return tree_unflatten(treedef, out), ClipPytreeAux(norm=res.norms[0], group_norms=group_norms)


def clip_pytree(
    pytree: Any,
    clipping_norm: float | PerGroup,
    return_zero: bool = False,
    *,
    compute_dtype: torch.dtype | None = None,
) -> tuple[Any, ClipPytreeAux]:
    """Clip one pytree to L2 norm ``clipping_norm`` (``_pytree.py:560-649``).

    Returns ``(clipped_pytree, ClipPytreeAux(norm, group_norms))``; ``norm`` is
    the float32 norm of the sanitised input.
    """
    return _scale_one(pytree, clipping_norm, _Kind("fixed"), return_zero=return_zero,
                      compute_dtype=compute_dtype)


def auto_scale_pytree(
    pytree: Any,
    R: float | PerGroup = 1.0,
    gamma: float = 0.01,
    *,
    compute_dtype: torch.dtype | None = None,
) -> tuple[Any, ClipPytreeAux]:
    """AUTO-S: scale one pytree by ``R / (||x|| + gamma)`` (``_pytree.py:422-507``)."""
    if gamma <= 0:
        raise ConfigurationError(f"gamma must be positive, got {gamma}")
    return _scale_one(pytree, R, _Kind("auto_s", float(gamma)), return_zero=False,
                      compute_dtype=compute_dtype)


__all__ = ["ClipPytreeAux", "auto_scale_pytree", "clip_pytree"]
