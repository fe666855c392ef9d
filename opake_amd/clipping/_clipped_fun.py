"""``clipped_fun`` / ``clipped_grad`` / ``auto_clipped_grad`` on the GPU.

Same call sites, return shapes and error classes as the reference
(packages/opake-engine/src/opake/api/engine/clipping/_clipped_fun.py:492-944,
_clipped_grad.py:86-362, _auto.py:211-367):

* per-example values come from ``torch.func.vmap`` over the batch arguments
  (for ``clipped_grad``: ``vmap(grad_and_value(loss_fn))``, the reference's
  ``_vmap_values``, _clipped_fun.py:476-489) on PyTorch-ROCm;
* the clip-and-sum of the stacked values runs in the HIP leaf kernels
  (``fused_stream_clip_and_sum``, the reference's streaming semantics,
  _streaming.py:39-185);
* ``x / normalize_by`` (_clipped_fun.py:880-883) and the ``ClippedPytree``
  metadata ``max_norm = C / normalize_by`` (_clipped_grad.py:220);
* ``microbatch_size`` accumulates chunk sums in float32 and casts once
  (``_microbatch_accumulate_reduced``, _clipped_fun.py:252-345);
* statistics count ``norm > C`` on the unguarded norms (:348-396).

* ``PerGroup`` clipping norms clip each group of leaves to its own bound by its
  own norm (``_streaming.py:63-104``); statistics are then counted per group
  (``_compute_clipping_stats``, :348-396) and ``clipping_rate`` in the aux is
  ``None``.

* ``second_moment=True`` adds the batch sum of the squared stored per-example
  values (``_streaming.py:167-172``) as a ``SecondMomentClippingOutput`` with
  ``max_norm = C^2 / normalize_by`` for the squared stream
  (``_clipped_fun.py:414-423``).

* leaves of float16, bfloat16, float32 or float64 (mixed), and
  ``compute_dtype`` (``_clipped_fun.py:91-170``, ``_pytree.py:84-108``) any of
  those four -- squares, guard roundoff and scale multiply in it
  (``promote(leaf, compute_dtype)``), batch sums in it and cast to the output
  dtype after, microbatch running sums in the wider of it and the output
  dtype; without one, the reference's defaults (float32 reductions for
  16-bit leaves, float64 when a leaf is float64).

* ``pre_clipping_transform`` (``_clipped_grad.py:97,285``, ``_auto.py:222``):
  applied to each example's gradient pytree inside the vmapped gradient
  function, and to the zero gradients of an empty batch.

Not covered (``OperationError``): custom scale functions, non-floating
leaves.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

import torch
from torch.autograd.profiler import record_function
from torch.func import grad_and_value, vmap

from opake_amd.clipping._leaves import (
    _group_layout,
    _sum_dtype_of,
    leaves_clip_sum,
    unsupported_reason,
)
from opake_amd.exceptions import ConfigurationError, InputTypeError, OperationError
from opake_amd.pytree import (
    tree_flatten,
    tree_flatten_with_paths,
    tree_leaves,
    tree_map,
    tree_unflatten,
)
from opake_amd.types import (
    ClippedPytree,
    ClipState,
    PerGroup,
    SecondMomentClippingOutput,
    clipped,
)

_DEFAULT_GAMMA = 0.01


@dataclass(frozen=True)
class FixedClipState(ClipState):
    """Marker state for fixed clipping (``_clipped_fun.py:36-42``)."""


@dataclass(frozen=True)
class AutoClipState(ClipState):
    """Marker state for AUTO-S scaling (``_auto.py``)."""


@dataclass(frozen=True)
class ClippedFunAux:
    """Per-example diagnostics of :func:`clipped_fun` (``_clipped_fun.py:52-80``)."""

    values: Any | None = None
    norms: Any | None = None
    clipped_norms: Any | None = None
    value_aux: Any | None = None
    clipping_rate: float | None = None
    batch_size: int = 0
    group_norms: dict | None = None


@dataclass(frozen=True)
class ClippingStats:
    """Aggregated statistics (``_clipped_fun.py:83-88``)."""

    num_clipped: float | dict
    clipping_rate: float | dict | None
    batch_size: int = 0


@dataclass(frozen=True)
class ClippedGradAux:
    """Diagnostics of :func:`clipped_grad` (``_clipped_grad.py:34-61``)."""

    loss_values: Any | None = None
    grad_norms: Any | None = None
    clipped_grad_norms: Any | None = None
    loss_aux: Any | None = None
    clipping_rate: float | None = None
    batch_size: int = 0
    group_norms: dict | None = None


@dataclass(frozen=True)
class _Scale:
    kind: str
    gamma: float = 0.0


def _to_tuple(x) -> tuple:
    return tuple(x) if isinstance(x, (tuple, list)) else (x,)


def _validate_clipping_norm(clipping_norm, name: str = "clipping_norm") -> None:
    """``_clipped_fun.py:194-207`` / ``_auto.py:99-108``."""
    if isinstance(clipping_norm, PerGroup):
        for group_name, value in clipping_norm.values.items():
            if value <= 0:
                raise ConfigurationError(
                    f"{name} must be positive for all groups, got {value} for group "
                    f"'{group_name}'")
        return
    if isinstance(clipping_norm, bool) or not isinstance(clipping_norm, (int, float)):
        raise InputTypeError(f"clipping_norm must be a float, got {type(clipping_norm)}")
    if clipping_norm <= 0:
        raise ConfigurationError(f"clipping_norm must be positive, got {clipping_norm}")


def _validate_static_args(argnums, batch_argnums, normalize_by) -> None:
    """``_clipped_grad.py:64-83``."""
    if normalize_by <= 0.0:
        raise ConfigurationError(f"normalize_by must be > 0, got {normalize_by}.")
    argnums, batch_argnums = _to_tuple(argnums), _to_tuple(batch_argnums)
    if not batch_argnums:
        raise ConfigurationError("Batch argnums must not be empty.")
    if min(argnums + batch_argnums) < 0:
        raise ConfigurationError(
            f"argnums={argnums} and batch_argnums={batch_argnums} must be >= 0.")
    shared = set(argnums) & set(batch_argnums)
    if shared:
        raise ConfigurationError(
            "Cannot compute clipped gradients for argnums that have a batch axis. "
            f"argnums={argnums} and batch_argnums={batch_argnums} with overlap {list(shared)}.")


def _batch_size(args, batch_argnums) -> int:
    for leaf in tree_leaves(args[batch_argnums[0]]):
        return int(leaf.shape[0])
    raise ConfigurationError("Could not determine the batch size from the batch arguments")


def _slice_args(args, batch_argnums, start, stop):
    return tuple(
        tree_map(lambda x: x[start:stop], a) if i in batch_argnums else a
        for i, a in enumerate(args)
    )


@dataclass
class _ChunkResult:
    reduced: Any
    norms: torch.Tensor
    post_sq: torch.Tensor | None
    nclipped: torch.Tensor  # [1], or [G] per group in sorted name order
    group_norms: dict | None
    storage: Any
    aux: Any = None
    squared: Any = None  # second moment: batch sums of the squared stored values


def _check_compute_dtype(compute_dtype):
    if compute_dtype is not None and not compute_dtype.is_floating_point:
        raise InputTypeError(
            f"compute_dtype must be a real floating-point dtype, got {compute_dtype!r}.  "
            "Integer/bool/complex compute dtypes can silently corrupt the L2-norm reduction "
            "(the squared sum is non-negative real and the final sqrt assumes a real "
            "accumulator).")


_ACCUMULATE = object()  # chunk sums of a microbatched call: the accumulation dtype


def _clip_sum_values(values, clipping_norm, scale, *, dtype, with_postsq,
                     second_moment=False, compute_dtype=None, output_dtype=None) -> _ChunkResult:
    """HIP clip-and-sum of a stacked pytree (``_streaming.py:39-185``).

    ``dtype``: the dtype of the batch sums (default: the leaf dtype); they are
    reduced in ``compute_dtype`` (float32 for 16-bit leaves without one) and
    cast to it (``_sum_clipped_tensor``, ``_clipped_fun.py:112-132``).
    ``dtype`` may be ``_ACCUMULATE``: each leaf's sum is then taken and kept in
    the microbatch accumulation dtype for the requested ``output_dtype``."""
    _check_compute_dtype(compute_dtype)
    grouped = isinstance(clipping_norm, PerGroup)
    if grouped:
        paths, leaves, treedef = tree_flatten_with_paths(values)
    else:
        leaves, treedef = tree_flatten(values)
    if not leaves:
        raise ConfigurationError("the clipped function returned no tensor leaves")
    B = leaves[0].shape[0]
    reason = unsupported_reason(leaves, clipping_norm, scale, compute_dtype=compute_dtype,
                                second_moment=False, batch_size=B)
    if reason is not None:
        raise OperationError(f"HIP clip-and-sum cannot serve this call: {reason}")
    if dtype is _ACCUMULATE:
        # Microbatch chunks: summed and kept in the accumulation dtype.
        sum_dtypes = {l.dtype: (_accumulation_dtype(l.dtype, output_dtype, compute_dtype),) * 2
                      for l in leaves}
    else:
        sum_dtypes = {l.dtype: (_sum_dtype_of(l.dtype, compute_dtype), dtype or l.dtype)
                      for l in leaves}
    detached = [l.detach() for l in leaves]
    names = None
    if grouped:
        names, leaf_groups, bounds = _group_layout(paths, clipping_norm)
        res = leaves_clip_sum(detached, bounds, kind=scale.kind, gamma=scale.gamma,
                              with_postsq=with_postsq, sum_dtypes=sum_dtypes,
                              leaf_groups=leaf_groups, second_moment=second_moment,
                              compute_dtype=compute_dtype)
    else:
        res = leaves_clip_sum(detached, float(clipping_norm), kind=scale.kind,
                              gamma=scale.gamma, with_postsq=with_postsq, sum_dtypes=sum_dtypes,
                              second_moment=second_moment, compute_dtype=compute_dtype)
    group_norms = None
    if grouped:
        group_norms = {n: res.group_norms[k] for k, n in enumerate(names)}
    return _ChunkResult(reduced=tree_unflatten(treedef, res.reduced), norms=res.norms,
                        post_sq=res.post_sq, nclipped=res.nclipped, group_norms=group_norms,
                        storage=tree_unflatten(treedef, [l.dtype for l in leaves]),
                        squared=(tree_unflatten(treedef, res.squared) if second_moment
                                 else None))


def _stats(nclipped: torch.Tensor, clipping_norm, batch_size: int):
    """Counts and rates, per group (sorted names) for ``PerGroup`` (:348-396)."""
    counts = nclipped.to(torch.float64).cpu().tolist()
    if isinstance(clipping_norm, PerGroup):
        names = sorted(clipping_norm.values)
        num = {n: float(c) for n, c in zip(names, counts)}
        rate = {n: c / max(1.0, float(batch_size)) for n, c in num.items()}
        return num, rate
    num = float(sum(counts))
    return num, num / max(1.0, float(batch_size))


def _accumulation_dtype(leaf_dtype, output_dtype, compute_dtype):
    """Microbatch sum dtype (``_accumulation_dtype``, ``_clipped_fun.py:135-148``)."""
    resolved = compute_dtype
    if resolved is None and leaf_dtype in (torch.float16, torch.bfloat16):
        resolved = torch.float32
    if output_dtype is None:
        return resolved if resolved is not None else leaf_dtype
    return torch.promote_types(resolved if resolved is not None else leaf_dtype, output_dtype)


def _make_clipped_fun(fun, has_aux, *, batch_argnums, clipping_norm, normalize_by, return_aux,
                      return_stats, microbatch_size, dtype, scale, state, second_moment=False,
                      compute_dtype=None):
    batch_argnums = _to_tuple(batch_argnums)
    if microbatch_size is not None and microbatch_size <= 0:
        raise ConfigurationError(f"microbatch_size must be positive, got {microbatch_size}")
    output_max_norm = clipping_norm / normalize_by
    squared_max_norm = (clipping_norm * clipping_norm) / normalize_by if second_moment else None

    def run_chunk(args, kwargs, out_dtype):
        in_dims = tuple(0 if i in batch_argnums else None for i in range(len(args)))
        if has_aux:
            values, aux = vmap(fun, in_dims=in_dims, out_dims=(0, 0), randomness="same")(
                *args, **kwargs)
        else:
            values = vmap(fun, in_dims=in_dims, out_dims=0, randomness="same")(*args, **kwargs)
            aux = None
        res = _clip_sum_values(values, clipping_norm, scale, dtype=out_dtype,
                               with_postsq=return_aux, second_moment=second_moment,
                               compute_dtype=compute_dtype, output_dtype=dtype)
        res.aux = aux
        return res

    def clipped_fn(*args, state, **kwargs):
        if len(args) <= max(batch_argnums):
            raise ConfigurationError("batch_argnums refers to a missing positional argument")
        B = _batch_size(args, batch_argnums)
        if B == 0:
            raise ConfigurationError(
                "Function-output clipping requires a non-empty batch because the output "
                "pytree cannot be inferred otherwise.")
        with torch.no_grad():
            if microbatch_size is None:
                res = run_chunk(args, kwargs, dtype)
                reduced, squared = res.reduced, res.squared
            else:
                # Chunk sums are accumulated in the wider of the compute and
                # output dtypes (float32 for bfloat16 leaves by default) and
                # cast once at the end (_microbatch_accumulate_reduced,
                # _clipped_fun.py:252-345).
                acc, acc_sq, parts = None, None, []
                for start in range(0, B, microbatch_size):
                    chunk = _slice_args(args, batch_argnums, start, min(B, start + microbatch_size))
                    r = run_chunk(chunk, kwargs, _ACCUMULATE)
                    acc = r.reduced if acc is None else tree_map(torch.add, acc, r.reduced)
                    if second_moment:
                        acc_sq = (r.squared if acc_sq is None
                                  else tree_map(torch.add, acc_sq, r.squared))
                    r.reduced = r.squared = None
                    parts.append(r)
                target = (parts[0].storage if dtype is None
                          else tree_map(lambda _: dtype, parts[0].storage))
                reduced = tree_map(lambda x, dt: x.to(dt), acc, target)
                squared = (tree_map(lambda x, dt: x.to(dt), acc_sq, target) if second_moment
                           else None)
                group_norms = None
                if parts[0].group_norms is not None:
                    group_norms = {n: torch.cat([p.group_norms[n] for p in parts])
                                   for n in parts[0].group_norms}
                aux = None
                if parts[0].aux is not None:
                    aux = tree_map(lambda *xs: torch.cat(xs), *[p.aux for p in parts])
                res = _ChunkResult(
                    reduced=reduced, norms=torch.cat([p.norms for p in parts]),
                    post_sq=torch.cat([p.post_sq for p in parts]) if return_aux else None,
                    nclipped=torch.stack([p.nclipped for p in parts]).sum(dim=0),
                    group_norms=group_norms, storage=parts[0].storage, aux=aux)
            if normalize_by != 1.0:
                reduced = tree_map(lambda x: x / normalize_by, reduced)
                if second_moment:
                    squared = tree_map(lambda x: x / normalize_by, squared)
        output = clipped(reduced, max_norm=output_max_norm)
        if second_moment:
            output = SecondMomentClippingOutput(
                grads=output, squared_grads=clipped(squared, max_norm=squared_max_norm))
        if not (return_aux or return_stats):
            return output, state
        num_clipped, rate = _stats(res.nclipped, clipping_norm, B)
        if return_aux:
            fun_aux = ClippedFunAux(
                values=res.aux, norms=res.norms, clipped_norms=torch.sqrt(res.post_sq),
                clipping_rate=rate if isinstance(rate, float) else None, batch_size=B,
                group_norms=res.group_norms)
            return (output, fun_aux), state
        return (output, ClippingStats(num_clipped=num_clipped, clipping_rate=rate,
                                      batch_size=B)), state

    return clipped_fn


def clipped_fun(
    fun: Callable[..., Any],
    has_aux: bool = False,
    *,
    batch_argnums: int | tuple[int, ...] = 0,
    clipping_norm: float = 1.0,
    normalize_by: float = 1.0,
    return_aux: bool = False,
    return_stats: bool = False,
    second_moment: bool = False,
    microbatch_size: int | None = None,
    dtype: torch.dtype | None = None,
    compute_dtype: torch.dtype | None = None,
):
    """Clip each example's output of ``fun`` to L2 norm ``clipping_norm`` and sum.

    Returns ``(clipped_fn, FixedClipState())``; ``clipped_fn(*args, state=)``
    returns ``(ClippedPytree, state)`` (``((ClippedPytree, aux), state)`` with
    ``return_aux`` / ``return_stats``).
    """
    if normalize_by <= 0.0:
        raise ConfigurationError(f"normalize_by must be > 0, got {normalize_by}.")
    if return_aux and return_stats:
        raise ConfigurationError("return_stats cannot be combined with return_aux=True")
    _validate_clipping_norm(clipping_norm)
    state = FixedClipState()
    fn = _make_clipped_fun(fun, has_aux, batch_argnums=batch_argnums, clipping_norm=clipping_norm,
                           normalize_by=normalize_by, return_aux=return_aux,
                           return_stats=return_stats, microbatch_size=microbatch_size,
                           dtype=dtype, scale=_Scale("fixed"), state=state,
                           second_moment=second_moment, compute_dtype=compute_dtype)
    return fn, state


def _identity(x):
    return x


def _grad_wrapper(loss_fn, argnums, has_aux, return_aux, pre_clipping_transform=_identity):
    """Per-example ``grad_and_value`` returning ``g`` or ``(g, {"values", "value_aux"})``;
    ``g`` is the per-example gradient after ``pre_clipping_transform``
    (``_clipped_grad.py:278-296``)."""
    gv = grad_and_value(loss_fn, argnums=argnums, has_aux=has_aux)

    def grad_fn(*args, **kwargs):
        g, out = gv(*args, **kwargs)
        g = pre_clipping_transform(g)
        if not return_aux:
            return g
        if has_aux:
            value, value_aux = out
            return g, {"values": value, "value_aux": value_aux}
        return g, {"values": out}

    return grad_fn


def _make_grad(loss_fn, argnums, has_aux, *, clipping_norm, normalize_by, batch_argnums,
               return_aux, return_stats, microbatch_size, dtype, scale, state,
               second_moment=False, compute_dtype=None, pre_clipping_transform=_identity):
    _validate_static_args(argnums, batch_argnums, normalize_by)
    if return_aux and return_stats:
        raise ConfigurationError("return_stats cannot be combined with return_aux=True")
    argnums_t = argnums if isinstance(argnums, int) else tuple(argnums)
    grad_fn = _grad_wrapper(loss_fn, argnums_t, has_aux, return_aux, pre_clipping_transform)
    inner = _make_clipped_fun(grad_fn, return_aux, batch_argnums=batch_argnums,
                              clipping_norm=clipping_norm, normalize_by=normalize_by,
                              return_aux=return_aux, return_stats=return_stats,
                              microbatch_size=microbatch_size, dtype=dtype, scale=scale,
                              state=state, second_moment=second_moment,
                              compute_dtype=compute_dtype)
    batch_t = _to_tuple(batch_argnums)
    max_norm = clipping_norm / normalize_by

    def wrapper(*args, state, **kwargs):
        if _batch_size(args, batch_t) == 0:
            # Zeros in the transformed gradient schema (empty_clipped_grads_like,
            # _helpers.py:95-122): the transform fixes structure, shape, device
            # and default dtype.
            template = pre_clipping_transform(tree_map(
                torch.zeros_like, args[argnums_t] if isinstance(argnums_t, int)
                else tuple(args[i] for i in argnums_t)))
            zeros = tree_map(lambda x: torch.zeros_like(x, dtype=dtype)
                             if isinstance(x, torch.Tensor) else x, template)
            grads = clipped(zeros, max_norm=max_norm)
            if second_moment:
                grads = SecondMomentClippingOutput(
                    grads=grads, squared_grads=clipped(
                        tree_map(torch.zeros_like, zeros),
                        max_norm=(clipping_norm * clipping_norm) / normalize_by))
            per_group = isinstance(clipping_norm, PerGroup)
            if return_aux:
                empty = torch.empty(0)
                return (grads, ClippedGradAux(loss_values=empty, grad_norms=empty,
                                              clipped_grad_norms=empty,
                                              clipping_rate=None if per_group else 0.0,
                                              batch_size=0)), state
            if return_stats:
                if per_group:
                    zeros_by_group = dict.fromkeys(sorted(clipping_norm.values), 0.0)
                    return (grads, ClippingStats(num_clipped=zeros_by_group,
                                                 clipping_rate=dict(zeros_by_group),
                                                 batch_size=0)), state
                return (grads, ClippingStats(num_clipped=0.0, clipping_rate=0.0,
                                             batch_size=0)), state
            return grads, state
        with record_function("opake::clipped_grad"):
            result, st = inner(*args, state=state, **kwargs)
        if not return_aux:
            return result, st
        grads, aux = result
        values = aux.values or {}
        return (grads, ClippedGradAux(
            loss_values=values.get("values"), grad_norms=aux.norms,
            clipped_grad_norms=aux.clipped_norms, loss_aux=values.get("value_aux"),
            clipping_rate=aux.clipping_rate, batch_size=aux.batch_size,
            group_norms=aux.group_norms)), st

    return wrapper


def clipped_grad(
    loss_fn: Callable,
    argnums: int | tuple[int, ...] = 0,
    has_aux: bool = False,
    *,
    clipping_norm: float,
    normalize_by: float = 1.0,
    batch_argnums: int | tuple[int, ...] = 1,
    return_aux: bool = False,
    return_stats: bool = False,
    second_moment: bool = False,
    pre_clipping_transform: Callable = _identity,
    microbatch_size: int | None = None,
    dtype: torch.dtype | None = None,
    compute_dtype: torch.dtype | None = None,
):
    """Sum of per-example clipped gradients of ``loss_fn`` (``_clipped_grad.py:86-362``).

    With ``second_moment`` the result is a ``SecondMomentClippingOutput``: the
    clipped sum and the sum of the squared clipped per-example gradients, with
    ``max_norm`` ``C / normalize_by`` and ``C^2 / normalize_by``.
    ``pre_clipping_transform`` maps each example's gradient pytree to the
    pytree that is clipped (e.g. a preconditioner scaling); ``compute_dtype``
    is the reduction dtype (float32, or bfloat16 with bfloat16 gradients).
    """
    _validate_clipping_norm(clipping_norm)
    state = FixedClipState()
    fn = _make_grad(loss_fn, argnums, has_aux, clipping_norm=clipping_norm,
                    normalize_by=normalize_by, batch_argnums=batch_argnums,
                    return_aux=return_aux, return_stats=return_stats,
                    microbatch_size=microbatch_size, dtype=dtype, scale=_Scale("fixed"),
                    state=state, second_moment=second_moment, compute_dtype=compute_dtype,
                    pre_clipping_transform=pre_clipping_transform)
    return fn, state


def auto_clipped_grad(
    loss_fn: Callable,
    argnums: int | tuple[int, ...] = 0,
    has_aux: bool = False,
    *,
    R: float = 1.0,
    gamma: float = _DEFAULT_GAMMA,
    normalize_by: float = 1.0,
    batch_argnums: int | tuple[int, ...] = 1,
    return_aux: bool = False,
    return_stats: bool = False,
    pre_clipping_transform: Callable = _identity,
    microbatch_size: int | None = None,
    dtype: Any = None,
    second_moment: bool = False,
):
    """AUTO-S: ``R * g_i / (||g_i|| + gamma)`` per example, summed (``_auto.py:211-367``);
    ``pre_clipping_transform`` as in :func:`clipped_grad`."""
    if isinstance(gamma, bool) or not isinstance(gamma, (int, float)) or not gamma > 0:
        raise ConfigurationError(f"gamma must be a positive float, got {gamma!r}")
    _validate_clipping_norm(R, "R")
    state = AutoClipState()
    fn = _make_grad(loss_fn, argnums, has_aux, clipping_norm=R, normalize_by=normalize_by,
                    batch_argnums=batch_argnums, return_aux=return_aux,
                    return_stats=return_stats, microbatch_size=microbatch_size, dtype=dtype,
                    scale=_Scale("auto_s", float(gamma)), state=state,
                    second_moment=second_moment, pre_clipping_transform=pre_clipping_transform)
    return fn, state


__all__ = [
    "AutoClipState",
    "ClippedFunAux",
    "ClippedGradAux",
    "ClippingStats",
    "FixedClipState",
    "auto_clipped_grad",
    "clipped_fun",
    "clipped_grad",
]
