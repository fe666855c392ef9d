"""CPU restatement of the reference's per-example clipping numerics.

TEST INFRASTRUCTURE: imported only by tests/, smoke() and bench.py's CPU
baseline.  Every function cites the reference code it restates
(``packages/opake-engine/src/opake/api/engine/clipping/``).  Computation uses
torch CPU tensors in the same dtypes and the same order of operations as the
reference, so float64 quantities match bit for bit and float32 / bf16 values
match up to the reduction order of ``torch.sum``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

REDUCTION_BLOCK = 2048  # _pytree.py:217 (_REDUCTION_BLOCK)
BLOCKED_REDUCTION_MIN = 4096  # _pytree.py:233 (_BLOCKED_REDUCTION_MIN)


def real_dtype(dtype: torch.dtype) -> torch.dtype:
    """_pytree.py:77-81."""
    if not dtype.is_complex:
        return dtype
    return torch.empty((), dtype=dtype).real.dtype


def resolve_compute_dtype_for_reduction(leaf_dtypes, compute_dtype=None) -> torch.dtype:
    """_pytree.py:84-108: explicit dtype wins; else fp32, widened by any
    float64 leaf (bf16/fp16 leaves count as fp32)."""
    if compute_dtype is not None:
        return compute_dtype
    acc = torch.float32
    for dt in leaf_dtypes:
        if not (dt.is_floating_point or dt.is_complex):
            continue
        r = real_dtype(dt)
        acc = torch.promote_types(acc, torch.float32 if r in (torch.float16, torch.bfloat16) else r)
    return acc


def guard_constants(storage_dtype, multiply_dtype, norm_roundoff: float) -> tuple[float, float]:
    """(relative, absolute) of ``_guard_scale`` (_pytree.py:111-141)."""
    store = torch.finfo(real_dtype(storage_dtype))
    mult = torch.finfo(real_dtype(multiply_dtype))
    if multiply_dtype == storage_dtype:
        rounding = store.eps
    else:
        rounding = store.eps / 2.0 + mult.eps
    return 1.0 - rounding - 2.0 * norm_roundoff, store.smallest_normal * store.eps


def finalize_scale(ratio, storage_dtype, multiply_dtype, norm_roundoff, *, clamp_to_one):
    """_pytree.py:144-157 on a float64 ratio tensor."""
    rel, absolute = guard_constants(storage_dtype, multiply_dtype, norm_roundoff)
    scale = ratio * rel - absolute
    if clamp_to_one:
        scale = torch.minimum(torch.ones_like(scale), scale)
    scale = torch.where(torch.isfinite(scale), scale, torch.zeros_like(scale))
    return torch.clamp(scale, min=0.0)


def scale_tensor(tensor, ratio, compute_dtype, norm_roundoff, *, clamp_to_one):
    """_pytree.py:160-204 for real floating leaves: multiply in
    promote(leaf, compute), cast once, zero sub-normals that rounded up."""
    multiply_dtype = torch.promote_types(tensor.dtype, compute_dtype)
    scale = finalize_scale(ratio, tensor.dtype, multiply_dtype, norm_roundoff,
                           clamp_to_one=clamp_to_one)
    scaled = tensor.to(multiply_dtype) * scale.to(multiply_dtype)
    stored = scaled.to(tensor.dtype)
    tiny = torch.finfo(stored.dtype).smallest_normal
    bad = (stored.abs() <= tiny) & (stored.abs() > scaled.abs())
    return torch.where(bad, torch.zeros_like(stored), stored)


def blocked_reduction_terms(n: int) -> int:
    """_pytree.py:242-249."""
    return REDUCTION_BLOCK + (n + REDUCTION_BLOCK - 1) // REDUCTION_BLOCK


def reduction_terms(numels) -> int:
    """_pytree.py:252-268, on per-example element counts."""
    widest = max([0, *numels])
    if widest <= 1:
        return 0
    if widest > BLOCKED_REDUCTION_MIN:
        return blocked_reduction_terms(widest)
    return widest


def norm_roundoff(acc_dtype, sq_dtype, n_leaves: int, n_reduction: int) -> float:
    """_pytree.py:271-283."""
    u_acc = torch.finfo(acc_dtype).eps / 2.0
    u_sq = torch.finfo(sq_dtype).eps / 2.0
    return (u_acc + (max(n_leaves, 1) + n_reduction) * u_sq) / 2.0


def leaf_sq_sum(leaf, acc_dtype, sq_dtype=torch.float64):
    """_pytree.py:286-314: square in acc_dtype, sum in sq_dtype, blocked by
    2048 above 4096 elements."""
    x = leaf.to(acc_dtype)
    flat = (x * x).reshape(-1)
    n = flat.shape[0]
    if n <= BLOCKED_REDUCTION_MIN:
        return flat.sum(dtype=sq_dtype)
    main = (n // REDUCTION_BLOCK) * REDUCTION_BLOCK
    total = flat[:main].reshape(-1, REDUCTION_BLOCK).sum(dim=-1, dtype=sq_dtype).sum(dtype=sq_dtype)
    if main < n:
        total = total + flat[main:].sum(dtype=sq_dtype)
    return total


def batched_leaf_sq_sum(leaf, acc_dtype, sq_dtype=torch.float64):
    """``vmap(_leaf_sq_sum)`` (_streaming.py:70-76) over the leading dim."""
    B = leaf.shape[0]
    x = leaf.to(acc_dtype)
    flat = (x * x).reshape(B, -1)
    n = flat.shape[1]
    if n <= BLOCKED_REDUCTION_MIN:
        return flat.sum(dim=1, dtype=sq_dtype)
    main = (n // REDUCTION_BLOCK) * REDUCTION_BLOCK
    total = flat[:, :main].reshape(B, -1, REDUCTION_BLOCK).sum(dim=-1, dtype=sq_dtype).sum(
        dim=1, dtype=sq_dtype)
    if main < n:
        total = total + flat[:, main:].sum(dim=1, dtype=sq_dtype)
    return total


def sanitize(t):
    return torch.nan_to_num(t, nan=0.0, posinf=0.0, neginf=0.0)


def conservative_bound(value: float) -> float:
    """_clipped_fun.py:206-216: float32(C), moved one ulp down when the
    rounding went up; returned as the float64 value the kernel path uses."""
    exact = float(value)
    bound = torch.tensor(exact)
    if bound.item() > exact:
        bound = torch.nextafter(bound, torch.full_like(bound, -math.inf))
    return float(bound.to(torch.float64))


@dataclass
class StreamResult:
    reduced: list  # per-leaf batch sums (in reduce dtype)
    norms: torch.Tensor  # float64 [B] (diagnostic norms before .to(acc))
    acc_dtype: torch.dtype
    clipped_norms: torch.Tensor | None
    group_norms: dict | None
    scales: dict  # storage dtype -> float64 scale [B]
    squared: list | None = None  # second moment: sum_b stored_b^2 per leaf


def stream_clip_and_sum(leaves, clipping_norm, *, kind="fixed", gamma=0.0, groups=None,
                        group_values=None, compute_dtype=None, reduce_dtype=None,
                        return_aux=False, second_moment=False) -> StreamResult:
    """_streaming.py:39-185 on a list of stacked leaves [B, *P].

    ``clipping_norm`` is the (already conservative) bound as a float; for
    per-group clipping pass ``groups`` (leaf index -> group name) and
    ``group_values`` (group name -> bound).  ``reduce_dtype`` maps a leaf dtype
    to the batch-sum output dtype (``_sum_clipped_tensor``,
    _clipped_fun.py:112-131): default keeps the leaf dtype with fp32
    accumulation for bf16/fp16.  ``second_moment`` also sums ``stored.square()``
    (squared in the leaf dtype, _streaming.py:167-172) into ``squared``.
    """
    B = leaves[0].shape[0] if leaves else 0
    acc = resolve_compute_dtype_for_reduction([l.dtype for l in leaves], compute_dtype)
    sq_dtype = torch.float64
    roundoff = norm_roundoff(acc, sq_dtype, len(leaves),
                             reduction_terms([l[0].numel() for l in leaves]))
    sq_norm = None
    group_sq = {}
    for i, leaf in enumerate(leaves):
        s = batched_leaf_sq_sum(sanitize(leaf), acc, sq_dtype)
        sq_norm = s if sq_norm is None else sq_norm + s
        if groups is not None:
            g = groups[i]
            group_sq[g] = group_sq[g] + s if g in group_sq else s
    if sq_norm is None:
        sq_norm = torch.zeros(B, dtype=sq_dtype)
    norm = torch.sqrt(sq_norm)

    def ratio_of(bound_value, nrm):
        bound = torch.clamp(torch.as_tensor(bound_value, dtype=nrm.dtype), min=0.0)
        if kind == "auto_s":
            return bound / (nrm + torch.as_tensor(gamma, dtype=nrm.dtype))
        return bound / nrm

    group_norms = None
    if groups is not None:
        group_norms = {g: torch.sqrt(v) for g, v in group_sq.items()}
        ratios = {g: ratio_of(group_values[g], n) for g, n in group_norms.items()}
    else:
        ratio = ratio_of(clipping_norm, norm)
    clamp = kind != "auto_s"

    post_sq = torch.zeros(B, dtype=acc) if return_aux else None
    reduced = []
    squared = []
    scales = {}
    for i, leaf in enumerate(leaves):
        r = ratios[groups[i]] if groups is not None else ratio
        shape = (B,) + (1,) * (leaf.dim() - 1)
        stored = scale_tensor(sanitize(leaf), r.reshape(shape), acc, roundoff, clamp_to_one=clamp)
        mult = torch.promote_types(leaf.dtype, acc)
        scales[leaf.dtype] = finalize_scale(r, leaf.dtype, mult, roundoff, clamp_to_one=clamp)
        if return_aux:
            x = stored.to(acc)
            post_sq = post_sq + (x * x).reshape(B, -1).sum(dim=1, dtype=acc)
        out_dtype = (reduce_dtype or {}).get(leaf.dtype, leaf.dtype)
        # _resolve_compute_dtype (_clipped_fun.py:91-111): an explicit
        # compute dtype, else float32 for float16 / bfloat16.
        accum = compute_dtype if compute_dtype is not None else (
            torch.float32 if leaf.dtype in (torch.float16, torch.bfloat16) else None)
        summed = torch.sum(stored, dim=0, dtype=accum)
        reduced.append(summed.to(out_dtype))
        if second_moment:
            squared.append(torch.sum(stored.square(), dim=0, dtype=accum).to(out_dtype))
    return StreamResult(
        reduced=reduced,
        norms=norm,
        acc_dtype=acc,
        clipped_norms=torch.sqrt(post_sq) if return_aux else None,
        group_norms=group_norms,
        scales=scales,
        squared=squared if second_moment else None,
    )


def num_clipped(norms_acc: torch.Tensor, clipping_norm: float) -> int:
    """_clipped_fun.py:348-396 (scalar C): strict ``norms > C`` on the
    diagnostic (acc-dtype) norms."""
    return int((norms_acc > clipping_norm).sum().item())


def normalize(x: torch.Tensor, normalize_by: float) -> torch.Tensor:
    """_clipped_fun.py:880-883."""
    return x / normalize_by if normalize_by != 1.0 else x


def clip_pytree_scalar(leaves, clipping_norm, compute_dtype=None):
    """``clip_pytree`` for one example (_pytree.py:560-649), list of leaves."""
    leaves = [sanitize(l) for l in leaves]
    acc = resolve_compute_dtype_for_reduction([l.dtype for l in leaves], compute_dtype)
    sq_dtype = torch.float64
    roundoff = norm_roundoff(acc, sq_dtype, len(leaves), reduction_terms([l.numel() for l in leaves]))
    sq = torch.zeros((), dtype=sq_dtype)
    for l in leaves:
        sq = sq + leaf_sq_sum(l, acc, sq_dtype)
    norm = torch.sqrt(sq)
    ratio = torch.clamp(torch.as_tensor(clipping_norm, dtype=norm.dtype), min=0.0) / norm
    out = [scale_tensor(l, ratio, acc, roundoff, clamp_to_one=True) for l in leaves]
    return out, norm.to(acc)


def auto_scale_scalar(leaves, R, gamma, compute_dtype=None):
    """``auto_scale_pytree`` for one example (_pytree.py:422-507)."""
    leaves = [sanitize(l) for l in leaves]
    acc = resolve_compute_dtype_for_reduction([l.dtype for l in leaves], compute_dtype)
    sq_dtype = torch.float64
    roundoff = norm_roundoff(acc, sq_dtype, len(leaves), reduction_terms([l.numel() for l in leaves]))
    sq = torch.zeros((), dtype=sq_dtype)
    for l in leaves:
        sq = sq + leaf_sq_sum(l, acc, sq_dtype)
    norm = torch.sqrt(sq)
    ratio = torch.clamp(torch.as_tensor(R, dtype=norm.dtype), min=0.0) / (
        norm + torch.tensor(gamma, dtype=norm.dtype))
    out = [scale_tensor(l, ratio, acc, roundoff, clamp_to_one=False) for l in leaves]
    return out, norm.to(acc)


__all__ = [
    "StreamResult",
    "auto_scale_scalar",
    "blocked_reduction_terms",
    "clip_pytree_scalar",
    "conservative_bound",
    "finalize_scale",
    "guard_constants",
    "leaf_sq_sum",
    "norm_roundoff",
    "normalize",
    "num_clipped",
    "reduction_terms",
    "resolve_compute_dtype_for_reduction",
    "sanitize",
    "scale_tensor",
    "stream_clip_and_sum",
]
