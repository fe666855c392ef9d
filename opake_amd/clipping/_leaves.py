"""Materialised-leaf clip-and-sum on the GPU: the fused-backend seam.

``fused_stream_clip_and_sum`` has the signature and return value of the
reference's streaming clip-and-sum
(packages/opake-engine/src/opake/api/engine/clipping/_streaming.py:39-185) and
of the backend that ``register_fused_clip_backend`` accepts
(``_kernel_backend.py:9-17``, consulted at ``_clipped_fun.py:442-467,680-692``).
It takes stacked per-example values ``[B, *P]`` and does the work in a fixed
number of HIP launches per storage dtype, whatever the number of leaves:

1. ``dpc_leaves_sqnorm``: per (example, leaf) fp64 sums of the squares of the
   sanitised values in the reduction dtype, 2048-element tiles, then
   ``dpc_row_sum_f64`` folds the leaves in flatten order (the reference's
   ``sq_norm = sq_0 + sq_1 + ...``);
2. ``dpc_clip_factors``: the guarded scale per storage dtype (fixed or AUTO-S),
   converted to that dtype's multiply dtype;
3. ``dpc_leaves_apply`` (float32 / bfloat16 leaves, float32 arithmetic) or
   ``dpc_leaves_apply_ex`` (every other combination): scale in the multiply
   dtype, one cast to the storage dtype, subnormals that rounded up zeroed,
   the batch sum in example order in the reduction dtype.

Leaves may be float16, bfloat16, float32 or float64, mixed; ``compute_dtype``
may be any of those four (the reference's reduction, multiply and sum dtypes
follow from it, ``_pytree.py:84-204``, ``_clipped_fun.py:91-148``).
Per-group clipping norms (``PerGroup``) clip each group to its own bound by
its own norm, with one scale row per group; ``second_moment`` adds the batch
sums of the squared stored values.  A call the kernels cannot take (leaves off
the GPU, non-floating leaves, leaves that need grad) goes to the ``fallback``
the caller registered with :func:`make_fused_backend` -- in the reference that
is its own PyTorch streaming path -- and raises ``OperationError`` when there
is none.
"""
from __future__ import annotations

import functools
import itertools
import math
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
_MAX_BATCH = 65535  # examples per launch (grid dimension of the leaf-sum pass)
KERNEL_DTYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float64)

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
    """Why the leaf kernels cannot serve this call, or ``None``.

    The kernels take stacked ``[B, *P]`` leaves of any of the four floating
    dtypes on one ROCm device, any floating ``compute_dtype`` among them, the
    fixed and AUTO-S scales, with or without the second moment."""
    kind = getattr(scale, "kind", "fixed")
    if kind not in ("fixed", "auto_s"):
        return f"scale kind {kind!r} has no kernel"
    if compute_dtype is not None and compute_dtype not in KERNEL_DTYPES:
        return f"no kernel computes in {compute_dtype}"
    if batch_size > _MAX_BATCH:
        return f"{batch_size} examples exceed the {_MAX_BATCH} one launch takes"
    odd = [type(x).__name__ for x in leaves if not isinstance(x, torch.Tensor)]
    if odd:
        return f"the values hold non-tensor leaves ({', '.join(sorted(set(odd)))})"
    devices = {x.device for x in leaves}
    if len(devices) > 1:
        return f"the leaves live on {len(devices)} devices"
    if devices and next(iter(devices)).type != "cuda":
        return f"the leaves live on {next(iter(devices))}, not on a ROCm device"
    foreign = {x.dtype for x in leaves} - set(KERNEL_DTYPES)
    if foreign:
        return f"no kernel stores {', '.join(sorted(map(str, foreign)))} leaves"
    if any(x.dim() == 0 or x.shape[0] != batch_size for x in leaves):
        return f"not every leaf is stacked along the batch of {batch_size}"
    if torch.is_grad_enabled() and any(x.requires_grad for x in leaves):
        return "leaves that require grad (the kernels record no autograd graph)"
    return None


def _sum_dtype_of(storage: torch.dtype, compute_dtype) -> torch.dtype:
    """Reduction dtype of a leaf's batch sum (``_resolve_compute_dtype``,
    ``_clipped_fun.py:91-110``): the compute dtype, else float32 for 16-bit
    storage, else the storage dtype."""
    if compute_dtype is not None:
        return compute_dtype
    return torch.float32 if storage in (torch.float16, torch.bfloat16) else storage


def probe_output_dtype(reduce_leaf, storage: torch.dtype, device) -> torch.dtype:
    """The dtype ``reduce_leaf`` returns for ``storage`` values: evaluated on
    the meta device (no data, no launch), on one element of the real device if
    the callable cannot run there."""
    try:
        return reduce_leaf(torch.empty((1, 1), dtype=storage, device="meta")).dtype
    except Exception:  # a callable that needs real data
        return reduce_leaf(torch.zeros((1, 1), dtype=storage, device=device)).dtype


@dataclass(frozen=True)
class _HostTiles:
    """One storage dtype's share of a leaf list, as host tables: which leaves
    (``members``, positions in the list), their per-example element counts,
    where each leaf's batch sum starts in the dtype's flat output, and the
    2048-element tiles (``tile_owner``: member index, ``tile_index``: tile
    number inside that leaf; ``first_tile``: each member's first tile)."""

    dtype: torch.dtype
    members: tuple
    numels: tuple
    out_starts: tuple
    total: int
    n_tiles: int
    first_tile: np.ndarray
    tile_owner: np.ndarray
    tile_index: np.ndarray


@functools.lru_cache(maxsize=64)
def _host_layout(signature: tuple) -> tuple:
    """Tile tables of a leaf list given as ``((dtype, numel), ...)``: they
    depend only on the element counts, not on the shapes."""
    parts = []
    for dtype in KERNEL_DTYPES:
        members = tuple(i for i, (dt, _) in enumerate(signature) if dt == dtype)
        if not members:
            continue
        numels = tuple(signature[i][1] for i in members)
        per_leaf = [-(-n // TILE) for n in numels]
        first = np.fromiter(itertools.accumulate(per_leaf, initial=0), dtype=np.int64,
                            count=len(per_leaf) + 1)
        owner = np.repeat(np.arange(len(numels), dtype=np.int32), per_leaf)
        index = (np.arange(first[-1], dtype=np.int64) - first[owner]).astype(np.int32)
        starts = tuple(itertools.accumulate(numels[:-1], initial=0))
        parts.append(_HostTiles(dtype=dtype, members=members, numels=numels, out_starts=starts,
                                total=sum(numels), n_tiles=int(first[-1]), first_tile=first,
                                tile_owner=owner, tile_index=index))
    return tuple(parts)


class _DeviceTiles:
    """A :class:`_HostTiles` with its tables on the device (content-cached
    device tables, so a HIP graph that captures a call keeps them alive)."""

    def __init__(self, host: _HostTiles, device):
        self.host = host
        self.dtype = host.dtype
        self.numel_t = device_table(host.numels, np.int64, device)
        self.out_start_t = device_table(host.out_starts, np.int64, device)
        self.column_t = device_table(host.members, np.int32, device)
        self.first_tile_t = device_table(host.first_tile, np.int64, device)
        self.tile_owner_t = device_table(host.tile_owner, np.int32, device)
        self.tile_index_t = device_table(host.tile_index, np.int32, device)


@dataclass
class LeafClipResult:
    """Outputs of :func:`leaves_clip_sum` (device tensors, nothing synchronised).

    ``reduced``: per-leaf batch sums.  ``norms``: [B] global norms in the
    reduction dtype.  ``post_sq``: float64 [B] ``||stored||^2`` or ``None``.
    ``nclipped``: int32 [1] examples with norm > C (global clipping) or [G] per
    group.  ``group_norms``: [G, B] (per-group clipping) or ``None``.
    ``scales``: float32 scale rows per storage dtype, [G, B] (G = 1 without
    groups), converted to that dtype's multiply dtype; ``scales64``: the
    float64 rows of the dtypes whose multiply dtype is float64.  ``squared``:
    per-leaf batch sums of the squared stored values (second moment) or
    ``None``.
    """

    reduced: list
    norms: torch.Tensor
    post_sq: torch.Tensor | None
    nclipped: torch.Tensor
    group_norms: torch.Tensor | None
    scales: dict
    squared: list | None = None
    scales64: dict | None = None


class LeafBatch:
    """Stacked per-example leaves ``[B, *P]`` prepared for the leaf kernels:
    the tile tables per storage dtype and the device pointer tables.  The
    leaves must stay alive (and unchanged) while the batch is in use."""

    def __init__(self, leaves):
        self.leaves = [l if l.is_contiguous() else l.contiguous() for l in leaves]
        self.device = self.leaves[0].device
        self.B = self.leaves[0].shape[0]
        self.L = len(self.leaves)
        signature = tuple((l.dtype, math.prod(l.shape[1:])) for l in self.leaves)
        self.parts = [_DeviceTiles(h, self.device) for h in _host_layout(signature)]
        self.ptr_tables = [pointer_table([self.leaves[i] for i in p.host.members], self.device)
                           for p in self.parts]

    @property
    def dtypes(self):
        return [p.dtype for p in self.parts]

    def sqnorms(self, acc_dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Per-leaf squared norms float64 [B, L] (``_leaf_sq_sum``: sanitised,
        converted to ``acc_dtype`` and squared there -- the reference's
        reduction dtype, any of the four floating dtypes -- summed in float64
        per 2048-element tile)."""
        B, L = self.B, self.L
        stream = nat.stream_handle(self.device)
        leaf_sq = torch.empty((B, L), dtype=torch.float64, device=self.device)
        for p, ptrs in zip(self.parts, self.ptr_tables):
            h = p.host
            partial = torch.empty((B, max(h.n_tiles, 1)), dtype=torch.float64, device=self.device)
            nat.call("dpc_leaves_sqnorm", nat.ptr(ptrs), nat.ptr(p.numel_t),
                     nat.ptr(p.tile_owner_t), nat.ptr(p.tile_index_t), nat.ptr(p.first_tile_t),
                     nat.ptr(p.column_t), len(h.members), h.n_tiles, B,
                     nat.dtype_code(p.dtype, wide=True), nat.dtype_code(acc_dtype, wide=True),
                     nat.ptr(partial), nat.ptr(leaf_sq), L, stream)
        return leaf_sq

    def apply(self, scale_rows: dict, leaf_rows=None, sum_dtypes=None, with_postsq=False,
              second_moment=False, mult_dtypes=None, scale64_rows=None):
        """Scale-store-sum over the batch: leaf l of storage dtype t uses row
        ``leaf_rows[l]`` (default 0) of ``scale_rows[t]`` (float32 [R, B],
        converted to t's multiply dtype ``mult_dtypes[t]``, default
        ``promote(t, float32)``; float64 multiplies read ``scale64_rows[t]``).
        ``sum_dtypes[t] = (A, O)``: the batch sum's reduction and output dtypes
        (default: :func:`_sum_dtype_of` and the storage dtype).  Returns
        ``(reduced, post_sq)`` (``post_sq`` float64 [B] or None), with
        ``second_moment`` also the batch sums of the squared stored values:
        ``(reduced, post_sq, squared)``."""
        B = self.B
        stream = nat.stream_handle(self.device)
        reduced = [None] * self.L
        squared = [None] * self.L
        post_sq = torch.zeros(B, dtype=torch.float64, device=self.device) if with_postsq else None
        for p, ptrs in zip(self.parts, self.ptr_tables):
            h, dtype = p.host, p.dtype
            acc, out_dtype = (sum_dtypes or {}).get(dtype, (_sum_dtype_of(dtype, None), dtype))
            mult = (mult_dtypes or {}).get(dtype, torch.promote_types(dtype, torch.float32))
            flat = torch.empty(h.total, dtype=out_dtype, device=self.device)
            flat_sq = torch.empty_like(flat) if second_moment else None
            leaf_row = None
            if leaf_rows is not None:
                leaf_row = device_table([leaf_rows[i] for i in h.members], np.int32, self.device)
            # The fp32 kernel: fp32 multiply and sum, output in the storage dtype or fp32.
            fast = (dtype in (torch.float32, torch.bfloat16) and mult == torch.float32
                    and acc == torch.float32 and out_dtype in (dtype, torch.float32))
            # Per (example, tile) partials of ||stored||^2, one per wave of the apply kernel.
            tile_sq = (torch.empty((B, 4 * h.n_tiles), device=self.device,
                                   dtype=torch.float32 if fast else torch.float64)
                       if with_postsq else None)
            if fast:
                nat.call("dpc_leaves_apply", nat.ptr(ptrs), nat.ptr(p.numel_t),
                         nat.ptr(p.tile_owner_t), nat.ptr(p.tile_index_t), nat.ptr(p.out_start_t),
                         h.n_tiles, B, nat.dtype_code(dtype), nat.ptr(scale_rows[dtype]),
                         nat.ptr(leaf_row), nat.ptr(flat), nat.ptr(flat_sq),
                         nat.dtype_code(out_dtype), nat.ptr(tile_sq), stream)
            else:
                rows64 = (scale64_rows or {}).get(dtype) if mult == torch.float64 else None
                if mult == torch.float64 and rows64 is None:
                    raise ConfigurationError("a float64 multiply needs the float64 scale rows")
                nat.call("dpc_leaves_apply_ex", nat.ptr(ptrs), nat.ptr(p.numel_t),
                         nat.ptr(p.tile_owner_t), nat.ptr(p.tile_index_t), nat.ptr(p.out_start_t),
                         h.n_tiles, B, nat.dtype_code(dtype, wide=True),
                         nat.dtype_code(mult, wide=True), nat.dtype_code(acc, wide=True),
                         nat.ptr(scale_rows[dtype]), nat.ptr(rows64), nat.ptr(leaf_row),
                         nat.ptr(flat), nat.ptr(flat_sq), nat.dtype_code(out_dtype, wide=True),
                         nat.ptr(tile_sq), stream)
            if with_postsq:
                post_sq += tile_sq.sum(dim=1, dtype=torch.float64)
            for j, i in enumerate(h.members):
                off, n = h.out_starts[j], h.numels[j]
                reduced[i] = flat[off:off + n].view(self.leaves[i].shape[1:])
                if second_moment:
                    squared[i] = flat_sq[off:off + n].view(self.leaves[i].shape[1:])
        if second_moment:
            return reduced, post_sq, squared
        return reduced, post_sq


def leaves_clip_sum(leaves, clipping_norm, *, kind: str = "fixed", gamma: float = 0.0,
                    with_postsq: bool = False, sum_dtypes=None, leaf_groups=None,
                    conservative: bool = True, second_moment: bool = False,
                    compute_dtype: torch.dtype | None = None):
    """Clip-and-sum of stacked leaves ``[B, *P]`` with the HIP kernels.

    ``clipping_norm`` is one bound, or -- with ``leaf_groups`` (group index of
    each leaf) -- a list of per-group bounds: each group is clipped to its own
    bound by its own norm (``_streaming.py:63-104``).  ``sum_dtypes[dtype] =
    (reduction dtype, output dtype)`` of the batch sums (default: the
    reference's reduction dtype for that storage dtype, output in the storage
    dtype).  ``conservative`` rounds each bound down to float32 first, as the
    reference's batch path does (``_clipped_fun.py:211-216``); the
    single-pytree functions use the exact bound (``_pytree.py:624-628``).
    ``compute_dtype`` (any of the four floating dtypes) is the reference's
    explicit reduction dtype (``_pytree.py:84-108``): squares in it, the
    guard's roundoff from it, and the scale multiply in ``promote(leaf dtype,
    compute_dtype)`` (``_pytree.py:160-187``).  See :class:`LeafClipResult`.
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
    mults = {dt: torch.promote_types(dt, acc) for dt in batch.dtypes}
    guards = [(*num.guard_constants(dt, mults[dt], roundoff), mults[dt]) for dt in batch.dtypes]
    scale_kind = nat.SCALE_AUTO_S if kind == "auto_s" else nat.SCALE_FIXED
    bound_of = num.conservative_bound if conservative else float
    if grouped:
        col_group = device_table(leaf_groups, np.int32, device)
        group_sq = torch.empty((n_groups, B), dtype=torch.float64, device=device)
        nat.call("dpc_group_sum_f64", nat.ptr(leaf_sq), B, L, L, 1, nat.ptr(col_group),
                 n_groups, nat.ptr(group_sq), 0, stream)
        cfs = [ops.clip_factors(group_sq[k], bound_of(bounds[k]), guards,
                                kind=scale_kind, gamma=gamma,
                                count_threshold=num.float32_of(bounds[k]))
               for k in range(n_groups)]
        # The clip kernel's norms are (float)sqrt(sq): the diagnostic when the
        # reduction dtype is float32 (_streaming.py:174-180).
        if acc == torch.float32:
            norms = torch.sqrt(sq).to(acc)
            group_norms = torch.stack([cf.norms for cf in cfs])
        else:
            norms = torch.sqrt(sq).to(acc)
            group_norms = torch.sqrt(group_sq).to(acc)
        nclipped = torch.cat([cf.nclipped for cf in cfs])
    else:
        cfs = [ops.clip_factors(sq, bound_of(bounds[0]), guards, kind=scale_kind,
                                gamma=gamma, count_threshold=num.float32_of(bounds[0]))]
        norms = cfs[0].norms if acc == torch.float32 else torch.sqrt(sq).to(acc)
        group_norms, nclipped = None, cfs[0].nclipped
    scales, scales64 = {}, {}
    for gi, dtype in enumerate(batch.dtypes):
        scales[dtype] = torch.stack([cf.scale[gi] for cf in cfs])
        if mults[dtype] == torch.float64:
            scales64[dtype] = torch.stack([cf.scale64[gi] for cf in cfs])
    if sum_dtypes is None:
        sum_dtypes = {dt: (_sum_dtype_of(dt, compute_dtype), dt) for dt in batch.dtypes}
    out = batch.apply(scales, leaf_groups if grouped else None, sum_dtypes, with_postsq,
                      second_moment=second_moment, mult_dtypes=mults, scale64_rows=scales64)
    reduced, post_sq = out[0], out[1]
    if post_sq is not None:
        post_sq = post_sq.to(acc)
    return LeafClipResult(reduced=reduced, norms=norms, post_sq=post_sq, nclipped=nclipped,
                          group_norms=group_norms, scales=scales,
                          squared=out[2] if second_moment else None,
                          scales64=scales64 or None)


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
        if reason is not None:
            if fallback is None:
                raise OperationError(f"HIP clip-and-sum cannot serve this call: {reason}")
            return fallback(values, clipping_norm, scale=scale, batch_size=batch_size,
                            reduce_leaf=reduce_leaf, compute_dtype=compute_dtype,
                            second_moment=second_moment, return_aux=return_aux,
                            return_stats=return_stats)
        device = leaves[0].device if leaves else torch.device("cuda")
        storage = sorted({l.dtype for l in leaves}, key=str)
        # One shared 0-d zero per storage dtype carries the leaves' dtypes.
        zero_of = {dt: torch.zeros((), dtype=dt, device=device) for dt in storage}
        grouped = isinstance(clipping_norm, PerGroup)
        names = None
        if not leaves or batch_size == 0:
            reduced = [reduce_leaf(l) for l in leaves]
            squared = [reduce_leaf(l) for l in leaves] if second_moment else None
            norms = torch.zeros(batch_size, dtype=torch.float32, device=device)
            post = norms.clone()
            group_norms = None
        else:
            # Batch sums: reduced in the reference's reduction dtype for the
            # storage dtype, returned in the dtype `reduce_leaf` produces.
            sum_dtypes = {dt: (_sum_dtype_of(dt, compute_dtype),
                               probe_output_dtype(reduce_leaf, dt, device)) for dt in storage}
            kind = getattr(scale, "kind", "fixed")
            gamma = float(getattr(scale, "gamma", 0.0))
            common = dict(kind=kind, gamma=gamma, with_postsq=return_aux, sum_dtypes=sum_dtypes,
                          second_moment=second_moment, compute_dtype=compute_dtype)
            if grouped:
                paths, _, _ = tree_flatten_with_paths(values)
                names, leaf_groups, bounds = _group_layout(paths, clipping_norm)
                res = leaves_clip_sum(leaves, bounds, leaf_groups=leaf_groups, **common)
            else:
                res = leaves_clip_sum(leaves, float(clipping_norm), **common)
            reduced, norms, post, group_norms = res.reduced, res.norms, res.post_sq, res.group_norms
            squared = res.squared
        diagnostics = {}
        if return_aux or return_stats:
            diagnostics["norms"] = norms.detach()
            if grouped and group_norms is not None:
                diagnostics["group_norms"] = {n: group_norms[k].detach() for k, n in enumerate(names)}
        if return_aux:
            diagnostics["clipped_norms"] = torch.sqrt(post).detach()
        markers = [zero_of[l.dtype] for l in leaves]
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
    "probe_output_dtype",
    "register_fused_clip_backend",
    "unsupported_reason",
]
