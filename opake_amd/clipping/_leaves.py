"""Materialised-leaf clip-and-sum on the GPU: the fused-backend seam.

``fused_stream_clip_and_sum`` has the signature and return value of the
reference's streaming clip-and-sum
(packages/opake-engine/src/opake/api/engine/clipping/_streaming.py:39-185) and
of the backend that ``register_fused_clip_backend`` accepts
(``_kernel_backend.py:9-17``, consulted at ``_clipped_fun.py:442-467,680-692``).
It takes stacked per-example values ``[B, *P]`` and does the work in a fixed
number of HIP launches per storage dtype, whatever the number of leaves:

1. ``dpc_leaves_sqnorm``: per (example, leaf) fp64 sums of fp32 squares of the
   sanitised values, 2048-element tiles, then ``dpc_row_sum_f64`` folds the
   leaves in flatten order (the reference's ``sq_norm = sq_0 + sq_1 + ...``);
2. ``dpc_clip_factors``: the guarded scale per storage dtype (fixed or AUTO-S);
3. ``dpc_leaves_apply``: scale in fp32, one cast to the storage dtype, bf16
   subnormals that rounded up zeroed, fp32 sum over the batch in example order.

Per-group clipping norms (``PerGroup``) clip each group to its own bound by
its own norm, with one scale row per group; ``second_moment`` adds the batch
sums of the squared stored values.  An explicit ``compute_dtype`` of float32,
or of bfloat16 with bfloat16 leaves, follows the reference's reduction and
multiply dtypes.  A call the kernels do not cover (another ``compute_dtype``,
dtypes other than float32 / bfloat16, leaves that need grad) goes to the
``fallback`` the caller registered with
:func:`make_fused_backend` -- in the reference that is its own PyTorch
streaming path -- and raises ``OperationError`` when there is none.
"""

from __future__ import annotations

import math
from collections import OrderedDict
from dataclasses import dataclass

import numpy as np
import torch

from opake_amd import _native as nat
from opake_amd._tables import device_table, pointer_table
from opake_amd import ops
from opake_amd.clipping import _numerics as num
from opake_amd.exceptions import ConfigurationError, OperationError
from opake_amd.pytree import (
    param_path,
    param_path_display,
    tree_flatten,
    tree_flatten_with_paths,
    tree_unflatten,
)
from opake_amd.types import PerGroup

TILE = 2048  # elements per tile: the reference's blocked-reduction width
_MAX_BATCH = 65535
_SUPPORTED = (torch.float32, torch.bfloat16)
_MAX_PLANS = 64

_fused_clip_backend = None


def register_fused_clip_backend(backend) -> None:
    """Register the fused clip-and-sum implementation (``_kernel_backend.py:9-12``)."""
    global _fused_clip_backend
    _fused_clip_backend = backend


def get_fused_clip_backend():
    """The registered implementation, if any (``_kernel_backend.py:15-17``)."""
    return _fused_clip_backend


def unsupported_reason(leaves, clipping_norm, scale, *, compute_dtype, second_moment,
                       batch_size) -> str | None:
    """Why the kernels cannot serve this call, or ``None``."""
    if getattr(scale, "kind", "fixed") not in ("fixed", "auto_s"):
        return f"unknown scale kind {scale.kind!r}"
    if compute_dtype is not None and compute_dtype != torch.float32:
        if compute_dtype != torch.bfloat16:
            return f"compute_dtype {compute_dtype} (supported: float32, or bfloat16 with " \
                   "bfloat16 leaves)"
        if any(isinstance(l, torch.Tensor) and l.dtype != torch.bfloat16 for l in leaves):
            return "compute_dtype bfloat16 needs bfloat16 leaves"
    if batch_size > _MAX_BATCH:
        return f"batch size {batch_size} exceeds {_MAX_BATCH}"
    grad_mode = torch.is_grad_enabled()
    for leaf in leaves:
        if not isinstance(leaf, torch.Tensor):
            return f"non-tensor leaf of type {type(leaf).__name__}"
        if not leaf.is_cuda:
            return f"leaf on device {leaf.device}, not a ROCm device"
        if leaf.device != leaves[0].device:
            return "the leaves span more than one device"
        if leaf.dtype not in _SUPPORTED:
            return f"leaf dtype {leaf.dtype} (supported: float32, bfloat16)"
        if grad_mode and leaf.requires_grad:
            return "a leaf requires grad"
        if leaf.dim() == 0 or leaf.shape[0] != batch_size:
            return "a leaf's leading dimension is not the batch"
    return None


def _output_dtypes(leaves, reduce_leaf):
    """Output dtype of ``reduce_leaf`` per storage dtype (the storage dtype or float32)."""
    out = {}
    for dtype in {leaf.dtype for leaf in leaves}:
        probe = reduce_leaf(torch.zeros((1,), dtype=dtype, device=leaves[0].device))
        if probe.dtype not in (dtype, torch.float32):
            return None
        out[dtype] = probe.dtype
    return out


_PLANS: OrderedDict = OrderedDict()


def _plan(leaves, device):
    """Tile tables per storage dtype, built on the host and copied once;
    cached by device and per-example shapes (bounded LRU)."""
    key = (device, tuple((leaf.dtype, tuple(leaf.shape[1:])) for leaf in leaves))
    plan = _PLANS.get(key)
    if plan is not None:
        _PLANS.move_to_end(key)
        return plan
    groups = []
    for dtype in (torch.bfloat16, torch.float32):
        idx = [i for i, leaf in enumerate(leaves) if leaf.dtype == dtype]
        if not idx:
            continue
        sizes = np.array([math.prod(leaves[i].shape[1:]) for i in idx], dtype=np.int64)
        tiles = (sizes + TILE - 1) // TILE
        tile_start = np.concatenate([[0], np.cumsum(tiles)]).astype(np.int64)
        tile_leaf = np.repeat(np.arange(len(idx), dtype=np.int32), tiles)
        tile_local = (np.arange(int(tile_start[-1]), dtype=np.int64) - tile_start[tile_leaf]).astype(
            np.int32)
        offsets = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)

        def dev(a):
            return torch.from_numpy(np.ascontiguousarray(a)).to(device)

        groups.append({
            "dtype": dtype,
            "idx": idx,
            "sizes_host": sizes.tolist(),
            "offsets_host": offsets.tolist(),
            "total": int(sizes.sum()),
            "n_tiles": int(tile_start[-1]),
            "sizes": dev(sizes),
            "out_offs": dev(offsets),
            "leaf_col": dev(np.array(idx, dtype=np.int32)),
            "tile_start": dev(tile_start),
            "tile_leaf": dev(tile_leaf),
            "tile_local": dev(tile_local),
        })
    plan = {"groups": groups, "n_leaves": len(leaves)}
    _PLANS[key] = plan
    if len(_PLANS) > _MAX_PLANS:
        _PLANS.popitem(last=False)
    return plan


_MARKERS: dict = {}


def _dtype_marker(leaf):
    key = (leaf.dtype, leaf.device)
    marker = _MARKERS.get(key)
    if marker is None:
        marker = _MARKERS[key] = leaf.new_zeros(())
    return marker


@dataclass
class LeafClipResult:
    """Outputs of :func:`leaves_clip_sum` (device tensors, nothing synchronised).

    ``reduced``: per-leaf batch sums.  ``norms``: float32 [B] global norms.
    ``post_sq``: float32 [B] ``||stored||^2`` or ``None``.  ``nclipped``:
    int32 [1] examples with norm > C (global clipping) or [G] per group.
    ``group_norms``: float32 [G, B] (per-group clipping) or ``None``.
    ``scales``: float32 scale rows per storage dtype, [G, B] (G = 1 without groups).
    ``squared``: per-leaf batch sums of the squared stored values (second
    moment) or ``None``.
    """

    reduced: list
    norms: torch.Tensor
    post_sq: torch.Tensor | None
    nclipped: torch.Tensor
    group_norms: torch.Tensor | None
    scales: dict
    squared: list | None = None


class LeafBatch:
    """Stacked per-example leaves ``[B, *P]`` prepared for the leaf kernels:
    the tile tables per storage dtype and the device pointer tables.  The
    leaves must stay alive (and unchanged) while the batch is in use."""

    def __init__(self, leaves):
        self.leaves = [l if l.is_contiguous() else l.contiguous() for l in leaves]
        self.device = self.leaves[0].device
        self.B = self.leaves[0].shape[0]
        self.L = len(self.leaves)
        self.plan = _plan(self.leaves, self.device)
        self.ptr_tables = [pointer_table([self.leaves[i] for i in g["idx"]], self.device)
                           for g in self.plan["groups"]]

    @property
    def dtypes(self):
        return [g["dtype"] for g in self.plan["groups"]]

    def sqnorms(self, acc_dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Per-leaf squared norms float64 [B, L] (``_leaf_sq_sum``: sanitised,
        squared in ``acc_dtype`` -- float32, or bfloat16 for bfloat16 leaves --
        summed in float64 per 2048-element tile)."""
        B, L = self.B, self.L
        stream = nat.stream_handle(self.device)
        leaf_sq = torch.empty((B, L), dtype=torch.float64, device=self.device)
        for g, ptrs in zip(self.plan["groups"], self.ptr_tables):
            partial = torch.empty((B, max(g["n_tiles"], 1)), dtype=torch.float64, device=self.device)
            nat.call("dpc_leaves_sqnorm", nat.ptr(ptrs), nat.ptr(g["sizes"]),
                     nat.ptr(g["tile_leaf"]), nat.ptr(g["tile_local"]), nat.ptr(g["tile_start"]),
                     nat.ptr(g["leaf_col"]), len(g["idx"]), g["n_tiles"], B,
                     nat.dtype_code(g["dtype"]), nat.dtype_code(acc_dtype), nat.ptr(partial),
                     nat.ptr(leaf_sq), L, stream)
        return leaf_sq

    def apply(self, scale_rows: dict, leaf_rows=None, out_dtypes=None, with_postsq=False,
              second_moment=False):
        """Scale-store-sum over the batch: leaf l of storage dtype t uses row
        ``leaf_rows[l]`` (default 0) of ``scale_rows[t]`` (float32 [R, B]).
        Returns ``(reduced, post_sq)``; ``post_sq`` is float32 [B] or None.
        With ``second_moment`` also the batch sums of the squared stored values:
        ``(reduced, post_sq, squared)``."""
        B = self.B
        stream = nat.stream_handle(self.device)
        reduced = [None] * self.L
        squared = [None] * self.L
        post_sq = torch.zeros(B, dtype=torch.float32, device=self.device) if with_postsq else None
        for g, ptrs in zip(self.plan["groups"], self.ptr_tables):
            dtype = g["dtype"]
            out_dtype = (out_dtypes or {}).get(dtype, dtype)
            flat = torch.empty(g["total"], dtype=out_dtype, device=self.device)
            flat_sq = torch.empty_like(flat) if second_moment else None
            # Four partials per tile (one per wave of the apply kernel).
            tile_sq = (torch.empty((B, 4 * g["n_tiles"]), dtype=torch.float32, device=self.device)
                       if with_postsq else None)
            rows = scale_rows[dtype]
            leaf_row = None
            if leaf_rows is not None:
                idx_rows = [leaf_rows[i] for i in g["idx"]]
                leaf_row = _device_table(self.device, ("leaf_row", dtype, tuple(idx_rows)),
                                         idx_rows, np.int32)
            nat.call("dpc_leaves_apply", nat.ptr(ptrs), nat.ptr(g["sizes"]),
                     nat.ptr(g["tile_leaf"]), nat.ptr(g["tile_local"]), nat.ptr(g["out_offs"]),
                     g["n_tiles"], B, nat.dtype_code(dtype), nat.ptr(rows), nat.ptr(leaf_row),
                     nat.ptr(flat), nat.ptr(flat_sq), nat.dtype_code(out_dtype), nat.ptr(tile_sq),
                     stream)
            if with_postsq:
                post_sq += tile_sq.sum(dim=1)
            for j, i in enumerate(g["idx"]):
                off, n = g["offsets_host"][j], g["sizes_host"][j]
                reduced[i] = flat[off:off + n].view(self.leaves[i].shape[1:])
                if second_moment:
                    squared[i] = flat_sq[off:off + n].view(self.leaves[i].shape[1:])
        if second_moment:
            return reduced, post_sq, squared
        return reduced, post_sq


def leaves_clip_sum(leaves, clipping_norm, *, kind: str = "fixed", gamma: float = 0.0,
                    with_postsq: bool = False, out_dtypes=None, leaf_groups=None,
                    conservative: bool = True, second_moment: bool = False,
                    compute_dtype: torch.dtype | None = None):
    """Clip-and-sum of stacked leaves ``[B, *P]`` with the HIP kernels.

    ``clipping_norm`` is one bound, or -- with ``leaf_groups`` (group index of
    each leaf) -- a list of per-group bounds: each group is clipped to its own
    bound by its own norm (``_streaming.py:63-104``).  Batch sums come out in
    ``out_dtypes[dtype]`` (default: the leaf dtype).  ``conservative`` rounds
    each bound down to float32 first, as the reference's batch path does
    (``_clipped_fun.py:211-216``); the single-pytree functions use the exact
    bound (``_pytree.py:624-628``).  ``compute_dtype`` (float32, or bfloat16
    with bfloat16 leaves) is the reference's explicit reduction dtype
    (``_pytree.py:84-108``): squares in it, the guard's roundoff from it, and
    the scale multiply in ``promote(leaf dtype, compute_dtype)`` (``_pytree.py:
    160-187``).  See :class:`LeafClipResult`.
    """
    batch = LeafBatch(leaves)
    device, B, L = batch.device, batch.B, batch.L
    grouped = leaf_groups is not None
    bounds = list(clipping_norm) if grouped else [clipping_norm]
    n_groups = len(bounds)
    stream = nat.stream_handle(device)
    acc = num.compute_dtype_for_reduction(batch.dtypes, compute_dtype)
    roundoff = num.norm_roundoff(acc, torch.float64, L,
                                 num.reduction_terms([math.prod(l.shape[1:]) for l in leaves]))
    leaf_sq = batch.sqnorms(acc)
    sq = torch.empty(B, dtype=torch.float64, device=device)
    nat.call("dpc_row_sum_f64", nat.ptr(leaf_sq), B, L, 0, nat.ptr(sq), stream)
    guards = []
    for dt in batch.dtypes:
        mult = torch.promote_types(dt, acc)
        guards.append((*num.guard_constants(dt, mult, roundoff), mult == torch.bfloat16))
    scale_kind = nat.SCALE_AUTO_S if kind == "auto_s" else nat.SCALE_FIXED
    bound_of = num.conservative_bound if conservative else float
    if grouped:
        col_group = _device_table(device, ("col_group", tuple(leaf_groups)), leaf_groups,
                                  np.int32)
        group_sq = torch.empty((n_groups, B), dtype=torch.float64, device=device)
        nat.call("dpc_group_sum_f64", nat.ptr(leaf_sq), B, L, L, nat.ptr(col_group), n_groups,
                 nat.ptr(group_sq), stream)
        cfs = [ops.clip_factors(group_sq[k], bound_of(bounds[k]), guards,
                                kind=scale_kind, gamma=gamma,
                                count_threshold=num.float32_of(bounds[k]))
               for k in range(n_groups)]
        norms = torch.sqrt(sq).to(torch.float32)
        group_norms = torch.stack([cf.norms for cf in cfs])
        nclipped = torch.cat([cf.nclipped for cf in cfs])
    else:
        cfs = [ops.clip_factors(sq, bound_of(bounds[0]), guards, kind=scale_kind,
                                gamma=gamma, count_threshold=num.float32_of(bounds[0]))]
        norms, group_norms, nclipped = cfs[0].norms, None, cfs[0].nclipped
    scales = {}
    for gi, dtype in enumerate(batch.dtypes):
        scales[dtype] = (torch.stack([cf.scale[gi] for cf in cfs]) if grouped
                         else cfs[0].scale[gi:gi + 1])
    out = batch.apply(scales, leaf_groups if grouped else None, out_dtypes, with_postsq,
                      second_moment=second_moment)
    reduced, post_sq = out[0], out[1]
    return LeafClipResult(reduced=reduced, norms=norms, post_sq=post_sq, nclipped=nclipped,
                          group_norms=group_norms, scales=scales,
                          squared=out[2] if second_moment else None)


def _device_table(device, key, values, np_dtype):
    """Small immutable index tables on the device (cached by content)."""
    return device_table(values, np_dtype, device)


def _group_layout(paths, clipping_norm):
    """Leaf -> group index (groups in sorted name order) and the group bounds.

    Requires a 1:1 match between leaf paths and the PerGroup's path keys
    (``_pytree.py:56-74``).
    """
    leaf_set = {param_path(p) for p in paths}
    group_set = set(clipping_norm.groups)
    if leaf_set != group_set:
        parts = ["PerGroup path keys must match the pytree tensor leaves exactly."]
        missing = sorted(leaf_set - group_set, key=param_path_display)
        extra = sorted(group_set - leaf_set, key=param_path_display)
        if missing:
            parts.append(f"Leaves with no group assignment: {missing}.")
        if extra:
            parts.append(f"Group paths with no matching leaf: {extra}.")
        raise ConfigurationError(" ".join(parts))
    names = sorted(clipping_norm.values)
    index = {n: k for k, n in enumerate(names)}
    leaf_groups = [index[clipping_norm.groups[param_path(p)]] for p in paths]
    bounds = [float(clipping_norm.values[n]) for n in names]
    return names, leaf_groups, bounds


def make_fused_backend(fallback=None):
    """A backend for :func:`register_fused_clip_backend`.

    ``fallback`` (the caller's own streaming implementation, same signature)
    serves calls the kernels do not support; without one they raise
    ``OperationError``.
    """

    def backend(values, clipping_norm, *, scale, batch_size, reduce_leaf, compute_dtype,
                second_moment, return_aux, return_stats):
        leaves, treedef = tree_flatten(values)
        reason = unsupported_reason(leaves, clipping_norm, scale, compute_dtype=compute_dtype,
                                    second_moment=second_moment, batch_size=batch_size)
        out_dtypes = None
        cast_to = None
        if reason is None and leaves and batch_size > 0:
            if compute_dtype == torch.bfloat16:
                # The reference sums in the compute dtype and casts after
                # (_sum_clipped_tensor, _clipped_fun.py:114-132).
                cast_to = {torch.bfloat16: reduce_leaf(
                    torch.zeros((1,), dtype=torch.bfloat16, device=leaves[0].device)).dtype}
            else:
                out_dtypes = _output_dtypes(leaves, reduce_leaf)
                if out_dtypes is None:
                    reason = "the requested output dtype is not supported"
        if reason is not None:
            if fallback is None:
                raise OperationError(f"HIP clip-and-sum cannot serve this call: {reason}")
            return fallback(values, clipping_norm, scale=scale, batch_size=batch_size,
                            reduce_leaf=reduce_leaf, compute_dtype=compute_dtype,
                            second_moment=second_moment, return_aux=return_aux,
                            return_stats=return_stats)
        kind = getattr(scale, "kind", "fixed")
        gamma = float(getattr(scale, "gamma", 0.0))
        grouped = isinstance(clipping_norm, PerGroup)
        names = None
        if not leaves or batch_size == 0:
            device = leaves[0].device if leaves else torch.device("cuda")
            reduced = [reduce_leaf(l) for l in leaves]
            squared = [reduce_leaf(l) for l in leaves] if second_moment else None
            norms = torch.zeros(batch_size, dtype=torch.float32, device=device)
            post = norms.clone()
            group_norms = None
        else:
            if grouped:
                paths, _, _ = tree_flatten_with_paths(values)
                names, leaf_groups, bounds = _group_layout(paths, clipping_norm)
                res = leaves_clip_sum(leaves, bounds, kind=kind, gamma=gamma,
                                      with_postsq=return_aux, out_dtypes=out_dtypes,
                                      leaf_groups=leaf_groups, second_moment=second_moment,
                                      compute_dtype=compute_dtype)
            else:
                res = leaves_clip_sum(leaves, float(clipping_norm), kind=kind, gamma=gamma,
                                      with_postsq=return_aux, out_dtypes=out_dtypes,
                                      second_moment=second_moment, compute_dtype=compute_dtype)
            reduced, norms, post, group_norms = res.reduced, res.norms, res.post_sq, res.group_norms
            squared = res.squared
            if cast_to is not None:
                reduced = [x.to(cast_to[l.dtype]) for x, l in zip(reduced, leaves)]
                if second_moment:
                    squared = [x.to(cast_to[l.dtype]) for x, l in zip(squared, leaves)]
        diagnostics = {}
        if return_aux or return_stats:
            diagnostics["norms"] = norms.detach()
            if grouped and group_norms is not None:
                diagnostics["group_norms"] = {n: group_norms[k].detach() for k, n in enumerate(names)}
        if return_aux:
            diagnostics["clipped_norms"] = torch.sqrt(post).detach()
        markers = [_dtype_marker(l) for l in leaves]
        return (
            tree_unflatten(treedef, reduced),
            tree_unflatten(treedef, markers),
            tree_unflatten(treedef, squared) if second_moment else (),
            tree_unflatten(treedef, markers) if second_moment else (),
            diagnostics if (return_aux or return_stats) else (),
        )

    return backend


fused_stream_clip_and_sum = make_fused_backend()


__all__ = [
    "fused_stream_clip_and_sum",
    "get_fused_clip_backend",
    "LeafClipResult",
    "leaves_clip_sum",
    "make_fused_backend",
    "register_fused_clip_backend",
    "unsupported_reason",
]
