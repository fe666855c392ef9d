"""Tensor-level wrappers of the native kernels.

Each function validates shapes on the host, allocates outputs and scratch with
torch on the inputs' device, and enqueues the kernels on the current stream.
None of them synchronises the host.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

import numpy as np

from opake_amd import _native as nat
from opake_amd._tables import device_table, pointer_table
from opake_amd.exceptions import ConfigurationError


def _contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _wants_error(out, err, return_error):
    """Whether a norm call writes its error bound.  Accumulating into ``out``
    without ``err`` drops the bound of the sum (``out + err`` would no longer
    bound the norm), so it must be asked for with ``return_error=False``."""
    if err is not None:
        if return_error is False:
            raise ConfigurationError("err was given together with return_error=False")
        return True
    if out is not None and return_error is None:
        raise ConfigurationError(
            "accumulating into `out` without `err` drops the rounding-error bound of the sum; "
            "pass the matching `err` vector, or return_error=False to accumulate the norms alone"
        )
    return bool(return_error)


def _error_out(err, B, dev, accumulate):
    """The error-bound vector of a norm call: ``err`` itself, or a new one."""
    if err is None:
        if accumulate:
            raise ConfigurationError("accumulating with an error bound needs its `err` vector")
        return torch.empty(B, dtype=torch.float64, device=dev)
    if err.dtype != torch.float64 or tuple(err.shape) != (B,) or not err.is_contiguous():
        raise ConfigurationError("err must be a contiguous float64 [B] vector")
    return err


def gram_sqnorms(
    A: torch.Tensor,
    G: torch.Tensor,
    *,
    with_bias: bool = False,
    out: torch.Tensor | None = None,
    err: torch.Tensor | None = None,
    return_error: bool | None = None,
):
    """``out[i] (+)= ||G_i^T A_i||_F^2 (+ ||sum_t G_i[t]||^2)`` in float64.

    ``A``: [B, T, din], ``G``: [B, T, dout], same dtype (bf16 or fp32).  When
    ``out`` is given the layer's contribution is added to it.  With ``err`` (or
    ``return_error=True``) the kernel also writes -- or, with ``out``, adds --
    an upper bound of the rounding error, so that ``out + err >=
    ||G_i^T A_i||^2`` exactly; the call then returns ``(out, err)``.
    Accumulating into ``out`` without ``err`` needs ``return_error=False``:
    the sum then carries no bound.
    """
    dev = nat.require_device(A, G, out, err)
    if A.dim() != 3 or G.dim() != 3 or A.shape[:2] != G.shape[:2]:
        raise ConfigurationError(
            f"expected A [B, T, din] and G [B, T, dout], got {tuple(A.shape)}, {tuple(G.shape)}"
        )
    if A.dtype != G.dtype:
        raise ConfigurationError("A and G must share a dtype")
    B, T, din = A.shape
    dout = G.shape[2]
    A, G = _contig(A), _contig(G)
    accumulate = out is not None
    with_err = _wants_error(out, err, return_error)
    if out is None:
        out = torch.empty(B, dtype=torch.float64, device=dev)
    elif out.dtype != torch.float64 or out.shape != (B,):
        raise ConfigurationError("out must be float64 [B]")
    if with_err:
        err = _error_out(err, B, dev, accumulate)
    if B > 0:
        ws_bytes = nat.load().dpc_gram_workspace_bytes(B, T)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        nat.call(
            "dpc_gram_sqnorms", nat.ptr(A), nat.ptr(G), B, T, din, dout,
            nat.dtype_code(A.dtype), int(with_bias), int(accumulate), nat.ptr(out),
            nat.ptr(err if with_err else None), nat.ptr(ws), ws_bytes, nat.stream_handle(dev),
        )
    return (out, err) if with_err else out


def gram_sqnorms_multi(
    A_list,
    G_list,
    *,
    out: torch.Tensor | None = None,
    err: torch.Tensor | None = None,
    return_error: bool | None = None,
):
    """``gram_sqnorms`` of several bias-free layers of one batch, summed over
    the layers in list order (``dpc_gram_sqnorms_multi``: one launch for all
    of them when they take the bf16 split path).  ``out`` / ``err`` as in
    :func:`gram_sqnorms`; the result equals consecutive ``gram_sqnorms``
    calls accumulating into the same ``out`` / ``err``."""
    n = len(A_list)
    if n == 0 or len(G_list) != n:
        raise ConfigurationError("expected matching, non-empty lists of A and G")
    dev = nat.require_device(*A_list, *G_list, out, err)
    dtype = A_list[0].dtype
    B, T = A_list[0].shape[:2]
    for A, G in zip(A_list, G_list):
        if A.dim() != 3 or G.dim() != 3 or A.shape[:2] != (B, T) or G.shape[:2] != (B, T):
            raise ConfigurationError("expected A [B, T, din], G [B, T, dout] with one B and T")
        if A.dtype != dtype or G.dtype != dtype:
            raise ConfigurationError("the layers' operands must share one dtype")
    accumulate = out is not None
    with_err = _wants_error(out, err, return_error)
    if out is None:
        out = torch.empty(B, dtype=torch.float64, device=dev)
    elif out.dtype != torch.float64 or out.shape != (B,):
        raise ConfigurationError("out must be float64 [B]")
    if with_err:
        err = _error_out(err, B, dev, accumulate)
    if B > 0:
        As = [_contig(A) for A in A_list]
        Gs = [_contig(G) for G in G_list]
        c_din = (ctypes.c_int * n)(*[A.shape[2] for A in As])
        c_dout = (ctypes.c_int * n)(*[G.shape[2] for G in Gs])
        ws_bytes = nat.load().dpc_gram_sqnorms_multi_workspace_bytes(
            n, c_din, c_dout, B, T, nat.dtype_code(dtype))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        vp = ctypes.c_void_p * n
        nat.call(
            "dpc_gram_sqnorms_multi", n, vp(*[t.data_ptr() for t in As]),
            vp(*[t.data_ptr() for t in Gs]), c_din, c_dout, B, T, nat.dtype_code(dtype),
            int(accumulate), nat.ptr(out), nat.ptr(err if with_err else None), nat.ptr(ws),
            ws_bytes, nat.stream_handle(dev),
        )
    return (out, err) if with_err else out


def flat_sqnorms(
    a: torch.Tensor,
    g: torch.Tensor,
    *,
    with_bias: bool = False,
    out: torch.Tensor | None = None,
    err: torch.Tensor | None = None,
    return_error: bool | None = None,
):
    """``out[i] (+)= ||a_i||^2 ||g_i||^2 (+ ||g_i||^2)`` for flat inputs [B, d];
    ``err`` / ``return_error`` as in :func:`gram_sqnorms`."""
    dev = nat.require_device(a, g, out, err)
    if a.dim() != 2 or g.dim() != 2 or a.shape[0] != g.shape[0] or a.dtype != g.dtype:
        raise ConfigurationError("expected a [B, din] and g [B, dout] of one dtype")
    B, din = a.shape
    dout = g.shape[1]
    accumulate = out is not None
    with_err = _wants_error(out, err, return_error)
    if out is None:
        out = torch.empty(B, dtype=torch.float64, device=dev)
    if with_err:
        err = _error_out(err, B, dev, accumulate)
    if B > 0:
        a, g = _contig(a), _contig(g)
        nat.call(
            "dpc_flat_sqnorms", nat.ptr(a), nat.ptr(g), B, din, dout, nat.dtype_code(a.dtype),
            int(with_bias), int(accumulate), nat.ptr(out), nat.ptr(err if with_err else None),
            nat.stream_handle(dev),
        )
    return (out, err) if with_err else out


@dataclass
class ClipFactors:
    """Outputs of :func:`clip_factors` (all on device, nothing synchronised)."""

    scale: torch.Tensor  # float32 [n_guards, B]
    norms: torch.Tensor  # float32 [B]
    nclipped: torch.Tensor  # int32 [1]
    plan: torch.Tensor  # uint8 [n_guards, plan bytes]: guard g's active example lists
    scale64: torch.Tensor | None = None  # float64 [n_guards, B] (guards with a float64 multiply)


def clip_factors(
    sqnorm: torch.Tensor,
    clipping_norm: float,
    guards: list[tuple[float, float]],
    *,
    err: torch.Tensor | None = None,
    kind: int = nat.SCALE_FIXED,
    gamma: float = 0.0,
    count_threshold: float,
    nonfinite: torch.Tensor | None = None,
) -> ClipFactors:
    """Guarded clip factors for each ``(rel, abs)`` guard, per example.

    A guard may carry a third element, its multiply dtype (``True`` means
    bfloat16): the scale is converted to it as ``scale.to(multiply_dtype)``
    does (float16 and bfloat16 through float32); with a float64 multiply the
    unconverted scale also comes back in ``scale64``.  ``err``
    (float64 [B], optional): the error bound of ``sqnorm``; the scale is then
    taken from ``sqrt(sqnorm + err)``, the reported norms and the clipped count
    from ``sqrt(sqnorm)``.  ``nonfinite`` (int32 [1], device or pinned host
    memory, optional) receives the number of examples whose ``sqnorm`` or
    ``err`` is not finite."""
    dev = nat.require_device(sqnorm, err)
    if sqnorm.dtype != torch.float64 or sqnorm.dim() != 1:
        raise ConfigurationError("sqnorm must be a float64 vector")
    if not 1 <= len(guards) <= 4:
        raise ConfigurationError("between 1 and 4 guards are supported")
    B = sqnorm.shape[0]
    if err is not None and (err.dtype != torch.float64 or tuple(err.shape) != (B,)):
        raise ConfigurationError("err must be a float64 vector like sqnorm")
    n = len(guards)
    rel = (ctypes.c_double * n)(*[g[0] for g in guards])
    abs_ = (ctypes.c_double * n)(*[g[1] for g in guards])
    mult, codes = _guard_mults(guards)
    cf = _clip_outputs(B, n, codes, dev)
    nat.call(
        "dpc_clip_factors", nat.ptr(_contig(sqnorm)), nat.ptr(None if err is None else _contig(err)),
        B, float(clipping_norm), kind, float(gamma), rel, abs_, mult, n, float(count_threshold),
        nat.ptr(cf.scale), nat.ptr(cf.scale64), nat.ptr(cf.norms), nat.ptr(cf.nclipped),
        nat.ptr(cf.plan), nat.ptr(nonfinite), nat.stream_handle(dev),
    )
    return cf


@dataclass
class ClipFactorGroups:
    """Outputs of :func:`clip_factors_groups`: group g's are ``group(g)``."""

    scale: torch.Tensor  # float32 [n_groups, n_guards, B]
    norms: torch.Tensor  # float32 [n_groups, B]
    nclipped: torch.Tensor  # int32 [n_groups]
    plan: torch.Tensor  # uint8 [n_groups, n_guards, plan bytes]
    scale64: torch.Tensor | None = None  # float64 [n_groups, n_guards, B]

    def group(self, g: int) -> ClipFactors:
        return ClipFactors(scale=self.scale[g], norms=self.norms[g],
                           nclipped=self.nclipped[g:g + 1], plan=self.plan[g],
                           scale64=None if self.scale64 is None else self.scale64[g])


def clip_factors_groups(
    sqnorm: torch.Tensor,
    clipping_norms: list[float],
    guards: list[tuple[float, float]],
    *,
    err: torch.Tensor | None = None,
    kind: int = nat.SCALE_FIXED,
    gamma: float = 0.0,
    count_thresholds: list[float],
    nonfinite: torch.Tensor | None = None,
) -> ClipFactorGroups:
    """:func:`clip_factors` for every row g of ``sqnorm`` (float64 [n_groups,
    B]) with its own bound ``clipping_norms[g]`` and count threshold, in one
    launch; the same bits as one call per group.  ``nonfinite``: int32
    [n_groups] (device or pinned host memory), one count per group."""
    dev = nat.require_device(sqnorm, err)
    if sqnorm.dtype != torch.float64 or sqnorm.dim() != 2:
        raise ConfigurationError("sqnorm must be a float64 [n_groups, B] tensor")
    G, B = sqnorm.shape
    if len(clipping_norms) != G or len(count_thresholds) != G:
        raise ConfigurationError("one clipping norm and count threshold per group")
    if not 1 <= len(guards) <= 4:
        raise ConfigurationError("between 1 and 4 guards are supported")
    if err is not None and (err.dtype != torch.float64 or tuple(err.shape) != (G, B)):
        raise ConfigurationError("err must be a float64 tensor like sqnorm")
    if nonfinite is not None and (nonfinite.dtype != torch.int32 or nonfinite.numel() < G):
        raise ConfigurationError("nonfinite must hold one int32 per group")
    n = len(guards)
    rel = (ctypes.c_double * n)(*[g[0] for g in guards])
    abs_ = (ctypes.c_double * n)(*[g[1] for g in guards])
    mult, codes = _guard_mults(guards)
    cs = (ctypes.c_double * G)(*[float(c) for c in clipping_norms])
    thr = (ctypes.c_float * G)(*[float(t) for t in count_thresholds])
    lib = nat.load()
    out = ClipFactorGroups(
        scale=torch.empty((G, n, B), dtype=torch.float32, device=dev),
        norms=torch.empty((G, B), dtype=torch.float32, device=dev),
        nclipped=torch.empty(G, dtype=torch.int32, device=dev),
        plan=torch.empty((G, n, lib.dpc_clip_plan_bytes(B)), dtype=torch.uint8, device=dev),
        scale64=(torch.empty((G, n, B), dtype=torch.float64, device=dev)
                 if nat.DPC_F64 in codes else None))
    nat.call(
        "dpc_clip_factors_groups", nat.ptr(_contig(sqnorm)),
        nat.ptr(None if err is None else _contig(err)), G, B, cs, kind, float(gamma), rel, abs_,
        mult, n, thr, nat.ptr(out.scale), nat.ptr(out.scale64), nat.ptr(out.norms),
        nat.ptr(out.nclipped), nat.ptr(out.plan), nat.ptr(nonfinite), nat.stream_handle(dev),
    )
    return out


def _guard_mults(guards):
    """The guards' multiply dtype codes (third element: a dtype, ``True`` for
    bfloat16, absent for float32) as a ctypes array, and as a list."""

    def code(g):
        m = g[2] if len(g) > 2 else torch.float32
        if isinstance(m, bool):
            m = torch.bfloat16 if m else torch.float32
        return nat.dtype_code(m, wide=True)

    codes = [code(g) for g in guards]
    return (ctypes.c_int * len(codes))(*codes), codes


def _clip_outputs(B, n, codes, dev) -> ClipFactors:
    return ClipFactors(
        scale=torch.empty((n, B), dtype=torch.float32, device=dev),
        norms=torch.empty(B, dtype=torch.float32, device=dev),
        nclipped=torch.empty(1, dtype=torch.int32, device=dev),
        plan=torch.empty((n, nat.load().dpc_clip_plan_bytes(B)), dtype=torch.uint8, device=dev),
        scale64=(torch.empty((n, B), dtype=torch.float64, device=dev)
                 if nat.DPC_F64 in codes else None))


# Counter buffers of dpc_gram_clip_factors, one per (device, stream), zero
# filled once: every call leaves them zero.
_GRAM_CLIP_COUNTERS: dict = {}


def _gram_clip_counters(dev, stream, nbytes: int) -> torch.Tensor:
    key = (str(dev), stream.value or 0)
    buf = _GRAM_CLIP_COUNTERS.get(key)
    if buf is None or buf.numel() * 4 < nbytes:
        buf = torch.zeros(max(1, (nbytes + 3) // 4), dtype=torch.int32, device=dev)
        _GRAM_CLIP_COUNTERS[key] = buf
    return buf


def gram_clip_factors(
    A: torch.Tensor,
    G: torch.Tensor,
    clipping_norm: float,
    guards,
    *,
    with_bias: bool = False,
    kind: int = nat.SCALE_FIXED,
    gamma: float = 0.0,
    count_threshold: float,
    nonfinite: torch.Tensor | None = None,
):
    """:func:`gram_sqnorms` (with its error bound) followed by
    :func:`clip_factors` on the result, in one launch where the split Gram
    kernel applies (``dpc_gram_clip_factors``; the same bits as the two
    calls).  Returns ``(sqnorm, err, ClipFactors)``.  Under HIP-graph capture
    the two calls run instead (the one-launch path keeps counters that live
    across calls)."""
    dev = nat.require_device(A, G)
    if A.dim() != 3 or G.dim() != 3 or A.shape[:2] != G.shape[:2] or A.dtype != G.dtype:
        raise ConfigurationError(
            f"expected A [B, T, din] and G [B, T, dout] of one dtype, got {tuple(A.shape)}, "
            f"{tuple(G.shape)}")
    if not 1 <= len(guards) <= 4:
        raise ConfigurationError("between 1 and 4 guards are supported")
    if torch.cuda.is_current_stream_capturing():
        sq, err = gram_sqnorms(A, G, with_bias=with_bias, return_error=True)
        cf = clip_factors(sq, clipping_norm, guards, err=err, kind=kind, gamma=gamma,
                          count_threshold=count_threshold, nonfinite=nonfinite)
        return sq, err, cf
    B, T, din = A.shape
    dout = G.shape[2]
    A, G = _contig(A), _contig(G)
    n = len(guards)
    rel = (ctypes.c_double * n)(*[g[0] for g in guards])
    abs_ = (ctypes.c_double * n)(*[g[1] for g in guards])
    mult, codes = _guard_mults(guards)
    cf = _clip_outputs(B, n, codes, dev)
    sq = torch.empty(B, dtype=torch.float64, device=dev)
    err = torch.empty(B, dtype=torch.float64, device=dev)
    if B > 0:
        stream = nat.stream_handle(dev)
        lib = nat.load()
        ws_bytes = lib.dpc_gram_clip_workspace_bytes(B, T)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        counters = _gram_clip_counters(dev, stream, lib.dpc_gram_clip_counter_bytes(B, T))
        nat.call(
            "dpc_gram_clip_factors", nat.ptr(A), nat.ptr(G), B, T, din, dout,
            nat.dtype_code(A.dtype), int(with_bias), float(clipping_norm), kind, float(gamma),
            rel, abs_, mult, n, float(count_threshold), nat.ptr(sq), nat.ptr(err),
            nat.ptr(cf.scale), nat.ptr(cf.scale64), nat.ptr(cf.norms), nat.ptr(cf.nclipped),
            nat.ptr(cf.plan), nat.ptr(nonfinite), nat.ptr(ws), ws_bytes, nat.ptr(counters),
            counters.numel() * 4, stream,
        )
    return sq, err, cf


@dataclass
class NoiseSpec:
    """Noise fused into an epilogue.

    ``mode``: ``NOISE_INJECTED`` (``noise`` holds float32 draws shaped like the
    output) or ``NOISE_PHILOX`` (device stream keyed by ``seed``/``leaf_id``).
    """

    sigma: float
    mode: int = nat.NOISE_PHILOX
    noise: torch.Tensor | None = None
    bias_noise: torch.Tensor | None = None
    seed: int = 0
    leaf_id: int = 0
    bias_leaf_id: int = 0


def clipped_sum(
    A: torch.Tensor,
    G: torch.Tensor,
    scale: torch.Tensor,
    *,
    plan: torch.Tensor | None = None,
    normalize_by: float = 1.0,
    noise: NoiseSpec | None = None,
    out_dtype: torch.dtype | None = None,
    with_bias: bool = False,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """``sum_i scale[i] G_i^T A_i`` (+ bias ``sum_i scale[i] sum_t G_i[t]``), then
    ``/ normalize_by`` and ``+ sigma * z`` in the epilogue.

    Returns ``(weight [dout, din], bias [dout] or None)`` in ``out_dtype``
    (default: the input dtype).
    """
    dev = nat.require_device(A, G, scale, plan)
    if A.dim() != 3 or G.dim() != 3 or A.shape[:2] != G.shape[:2] or A.dtype != G.dtype:
        raise ConfigurationError("expected A [B, T, din], G [B, T, dout] of one dtype")
    B, T, din = A.shape
    dout = G.shape[2]
    if scale.dtype != torch.float32 or scale.numel() < B:
        raise ConfigurationError("scale must be float32 with B entries")
    out_dtype = out_dtype or A.dtype
    A, G = _contig(A), _contig(G)
    out = torch.empty((dout, din), dtype=out_dtype, device=dev)
    bias_out = torch.empty(dout, dtype=out_dtype, device=dev) if with_bias else None
    ws_bytes = nat.load().dpc_clipped_sum_workspace_bytes(B, T, din, dout, nat.dtype_code(A.dtype))
    # The workspace holds the bias partials and, for launches of few output
    # tiles, the split-K slices.
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if ws_bytes else None
    spec = noise or NoiseSpec(sigma=0.0, mode=nat.NOISE_NONE)
    if spec.sigma != 0.0 and spec.mode == nat.NOISE_INJECTED:
        for t, shape in ((spec.noise, (dout, din)), (spec.bias_noise, (dout,))):
            if t is None and shape == (dout,) and not with_bias:
                continue
            if t is None or t.dtype != torch.float32 or tuple(t.shape) != shape or not t.is_cuda:
                raise ConfigurationError(f"injected noise must be float32 {shape} on the device")
    nat.call(
        "dpc_clipped_sum", nat.ptr(A), nat.ptr(G), nat.ptr(_contig(scale)), nat.ptr(plan), B, T,
        din, dout, nat.dtype_code(A.dtype), float(normalize_by), spec.mode,
        nat.ptr(spec.noise), nat.ptr(spec.bias_noise), spec.seed & ((1 << 64) - 1),
        spec.leaf_id & 0xFFFFFFFF, spec.bias_leaf_id & 0xFFFFFFFF, float(spec.sigma), nat.dtype_code(out_dtype), nat.ptr(out),
        int(with_bias), nat.ptr(bias_out), nat.ptr(ws), ws_bytes if ws is not None else 0,
        nat.stream_handle(dev),
    )
    return out, bias_out


def clipped_sum_multi(
    A_list,
    G_list,
    scale: torch.Tensor,
    *,
    plan: torch.Tensor | None = None,
    normalize_by: float = 1.0,
    noises: list[NoiseSpec | None] | None = None,
    out_dtype: torch.dtype | None = None,
) -> list[torch.Tensor]:
    """``clipped_sum`` of several bias-free layers of one clipping group (the
    same examples, ``scale`` and ``plan``) -- ``dpc_clipped_sum_multi``: on the
    bf16 MFMA path the layers' output tiles share launches.  ``noises[i]``:
    layer i's noise (None: none); the specs must share one mode and seed.
    Returns one [dout, din] tensor per layer.  When every layer takes the
    MFMA path (bf16, T % 64 == 0, widths % 8 == 0, a plan) each result equals
    its own ``clipped_sum`` call without a split-K workspace; otherwise the
    layers run as their own ``clipped_sum`` calls."""
    n = len(A_list)
    if n == 0 or len(G_list) != n:
        raise ConfigurationError("expected matching, non-empty lists of A and G")
    dev = nat.require_device(*A_list, *G_list, scale, plan)
    dtype = A_list[0].dtype
    B, T = A_list[0].shape[:2]
    for A, G in zip(A_list, G_list):
        if A.dim() != 3 or G.dim() != 3 or A.shape[:2] != (B, T) or G.shape[:2] != (B, T):
            raise ConfigurationError("expected A [B, T, din], G [B, T, dout] with one B and T")
        if A.dtype != dtype or G.dtype != dtype:
            raise ConfigurationError("the layers' operands must share one dtype")
    if scale.dtype != torch.float32 or scale.numel() < B:
        raise ConfigurationError("scale must be float32 with B entries")
    noises = list(noises) if noises is not None else [None] * n
    if len(noises) != n:
        raise ConfigurationError("expected one noise spec (or None) per layer")
    live = [sp for sp in noises if sp is not None and sp.sigma != 0.0]
    mode = live[0].mode if live else nat.NOISE_NONE
    seed = live[0].seed if live else 0
    if any(sp.mode != mode or sp.seed != seed or sp.bias_noise is not None for sp in live):
        raise ConfigurationError("the layers' noise specs must share one mode and seed, no bias")
    out_dtype = out_dtype or dtype
    mfma = plan is not None and B > 0 and dtype == torch.bfloat16 and T % 64 == 0 and all(
        A.shape[2] % 8 == 0 and G.shape[2] % 8 == 0
        and B * T * max(A.shape[2], G.shape[2]) * 2 < 2 ** 31 for A, G in zip(A_list, G_list))
    if not mfma:
        return [clipped_sum(A, G, scale, plan=plan, normalize_by=normalize_by, noise=sp,
                            out_dtype=out_dtype)[0] for A, G, sp in zip(A_list, G_list, noises)]
    As = [_contig(A) for A in A_list]
    Gs = [_contig(G) for G in G_list]
    dins = [A.shape[2] for A in As]
    douts = [G.shape[2] for G in Gs]
    outs = [torch.empty((o, i), dtype=out_dtype, device=dev) for i, o in zip(dins, douts)]
    sig = [sp.sigma if sp is not None else 0.0 for sp in noises]
    zs = []
    for sp, o, i in zip(noises, douts, dins):
        z = None
        if sp is not None and sp.sigma != 0.0 and mode == nat.NOISE_INJECTED:
            z = sp.noise
            if z is None or z.dtype != torch.float32 or tuple(z.shape) != (o, i) or not z.is_cuda:
                raise ConfigurationError(f"injected noise must be float32 {(o, i)} on the device")
            z = _contig(z)
        zs.append(z)
    vp = ctypes.c_void_p * n
    nat.call(
        "dpc_clipped_sum_multi", n, vp(*[t.data_ptr() for t in As]), vp(*[t.data_ptr() for t in Gs]),
        (ctypes.c_int * n)(*dins), (ctypes.c_int * n)(*douts), nat.ptr(_contig(scale)),
        nat.ptr(plan), B, T, nat.dtype_code(dtype), float(normalize_by), mode,
        vp(*[z.data_ptr() if z is not None else None for z in zs]), seed & ((1 << 64) - 1),
        (ctypes.c_uint32 * n)(*[(sp.leaf_id if sp is not None else 0) & 0xFFFFFFFF
                                for sp in noises]),
        (ctypes.c_double * n)(*sig), nat.dtype_code(out_dtype),
        vp(*[t.data_ptr() for t in outs]), nat.stream_handle(dev),
    )
    return outs


_GRAM_TILE = 128  # rows of a Gram tile of the grouped norm kernel
_GRAM_REC_WORDS = 12  # float64 words of a Gram work item's record
_STEP_ROWS = 64  # rows of a K step of the grouped clipped sum


def _xcd_cus(device) -> int:
    """CUs per XCD of a ROCm device (8 XCDs; 32 CUs each on MI355X)."""
    dev = torch.device(device)
    if dev.type != "cuda" or not torch.cuda.is_available():
        return 32
    return max(1, torch.cuda.get_device_properties(dev).multi_processor_count // 8)


class SegmentLayout:
    """Rows of E problems cut into per-example segments, built on the host.

    ``lengths[e][k]`` is the number of rows of segment k of problem e; problem
    e's rows are its segments in order.  Segment ``v = e * K + k`` (K segments
    per problem, e.g. K = batch size).  ``gram_weights[e]`` (default 1) is the
    relative cost of a Gram tile pair of problem e (its din + dout): the Gram
    work items are issued most expensive first, so that a launch over problems
    of different widths ends evenly.  ``gram_dims[e]`` (optional) is problem
    e's (din, dout), which prices the grouped split kernel's items (one per
    operand) more exactly.  The device tables (segment first rows and
    lengths, Gram work items) are copied in one transfer.

    Two Gram schedules are kept: tile-pair items for every segment (any
    dtype), and for the bf16 MFMA path the split kernel's items -- two per
    segment of 1 .. 320 rows (A and G) -- with tile-pair items for the
    longer segments only.
    """

    MAX_GRAM_PROBLEMS = 64
    XCDS = 8
    SPLIT_MAX_ROWS = 320  # segments the grouped split kernel takes (10 units of 32 rows)

    @classmethod
    def _split_schedule(cls, seg, seg_len, seg_row0, seg_group, seg_first, k_op):
        """Items of the grouped split kernel for segments `seg`: per segment
        (a "set") the A item and the G item, (problem | op << 8 | set << 9,
        first row, rows, first record slot).  Sets go whole to the 8 XCD bins,
        most expensive first in snake order (both items of a set on one XCD,
        where they meet through its L2); within a bin the items run most
        expensive first.  Returns the padded [8 * per, 4] table."""
        import numpy as np

        n_sets = len(seg)
        if n_sets == 0:
            return np.zeros((0, 4), dtype=np.int64)
        rows = seg_len[seg]
        blocks = np.where(rows > 288, 55, np.where(rows > 256, 45, 36))  # 32 x 32 blocks
        prob = seg_group[seg]
        cost = np.stack([k_op[prob, 0] * blocks, k_op[prob, 1] * blocks], axis=1)
        order = np.argsort(-cost.sum(axis=1), kind="stable")
        r = np.arange(n_sets)
        lap, pos = r // cls.XCDS, r % cls.XCDS
        bin_of = np.empty(n_sets, dtype=np.int64)
        bin_of[order] = np.where(lap % 2 == 0, pos, cls.XCDS - 1 - pos)
        per = 2 * int(np.bincount(bin_of, minlength=cls.XCDS).max())
        words = np.stack([
            np.stack([prob | (op << 8) | (np.arange(n_sets) << 9), seg_row0[seg], rows,
                      seg_first[seg]], axis=1)
            for op in (0, 1)], axis=1)  # [n_sets, 2, 4]
        out = np.zeros((cls.XCDS * per, 4), dtype=np.int64)
        out[:, 0] = -1
        for x in range(cls.XCDS):
            sets = np.nonzero(bin_of == x)[0]
            if not len(sets):
                continue
            it = words[sets].reshape(-1, 4)
            c = cost[sets].reshape(-1)
            it = it[np.argsort(-c, kind="stable")]
            out[x * per:x * per + len(it)] = it
        return out

    @classmethod
    def _xcd_schedule(cls, items, cost, seg_of_item, item_start, xcd_cus=32):
        """Order Gram items for the kernel's XCD placement (item l of a launch of
        8 * per runs on XCD l // per): segments go whole to the 8 bins, most
        expensive first in snake order, so each XCD gets a balanced share and
        keeps a segment's tile pairs (which re-read the same rows) together in
        its L2.
        Within a bin, hardware hands the items to the XCD's CUs in turn, so
        with n items on C CUs (C < n <= 2 C) the items at positions k and C + k
        share CU k: the 2 (n - C) lightest items take those positions (first
        and last) and the rest the middle; otherwise the bin runs segment by
        segment.  Bins are padded to equal length with empty items (problem
        field -1)."""
        import numpy as np

        n_seg = len(item_start) - 1
        counts = np.diff(item_start)
        seg_cost = np.bincount(seg_of_item, weights=cost, minlength=n_seg)
        # Segments with items, most expensive first, dealt to the bins in
        # snake order (0..7, 7..0, ...): balanced to within one segment.
        order = np.argsort(-seg_cost, kind="stable")
        order = order[counts[order] > 0]
        r = np.arange(len(order))
        lap, pos = r // cls.XCDS, r % cls.XCDS
        seg_bin = np.where(lap % 2 == 0, pos, cls.XCDS - 1 - pos)
        per = int(np.bincount(seg_bin, weights=counts[order], minlength=cls.XCDS).max()) \
            if len(order) else 0
        out = np.zeros((cls.XCDS * per, 4), dtype=np.int64)
        out[:, 0] = -1
        for x in range(cls.XCDS):
            segs = order[seg_bin == x]  # most expensive first
            if not len(segs):
                continue
            lens = counts[segs]
            first = np.repeat(item_start[segs] - (np.cumsum(lens) - lens), lens)
            idx = first + np.arange(int(lens.sum()))
            n = len(idx)
            a = n - xcd_cus
            if 0 < a and n <= 2 * xcd_cus:
                by_cost = idx[np.argsort(cost[idx], kind="stable")]
                light, heavy = by_cost[:2 * a], by_cost[2 * a:][::-1]
                idx = np.concatenate([light[:a], heavy, light[a:]])
            out[x * per:x * per + n] = items[idx]
        return out

    def __init__(self, lengths, device, gram_weights=None, gram_dims=None):
        import numpy as np

        lens = np.asarray(lengths, dtype=np.int64)
        if lens.ndim != 2 or (lens < 0).any():
            raise ConfigurationError("segment lengths must be a non-negative [E, K] table")
        self.E, self.K = lens.shape
        self.S = self.E * self.K
        self.lengths = lens
        self.rows = lens.sum(axis=1)
        self.max_rows = int(self.rows.max()) if self.E else 0
        if self.max_rows >= 1 << 30:
            raise ConfigurationError("too many rows in one problem")
        weights = np.ones(self.E) if gram_weights is None else np.asarray(gram_weights, float)
        flat = lens.reshape(-1)
        row0 = (np.cumsum(lens, axis=1) - lens).reshape(-1)
        group = np.repeat(np.arange(self.E, dtype=np.int64), self.K)
        nt = (flat + _GRAM_TILE - 1) // _GRAM_TILE
        npairs = nt * (nt + 1) // 2
        if npairs.size and npairs.max() >= 1 << 16:
            raise ConfigurationError("a segment is too long for the grouped Gram kernel")
        item_start = np.concatenate([[0], np.cumsum(npairs)])
        self.n_items = int(item_start[-1])
        seg_of_item = np.repeat(np.arange(self.S), npairs)
        pair = np.arange(self.n_items) - item_start[seg_of_item]
        # Cost of a pair: the problem's weight times the live 32-row blocks of
        # both tiles (blocks past the segment's end are skipped).
        q = ((np.sqrt(8 * pair + 1) - 1) // 2).astype(np.int64)
        q = np.where((q + 1) * (q + 2) // 2 <= pair, q + 1, q)
        pp = pair - q * (q + 1) // 2
        seg_len = flat[seg_of_item]

        def live_rows(t):
            rows = np.clip(seg_len - t * _GRAM_TILE, 0, _GRAM_TILE)
            return (rows + 31) // 32

        cost = weights[group[seg_of_item]] * live_rows(pp) * live_rows(q)
        slot = np.arange(self.n_items)
        items = np.stack([(group[seg_of_item] << 16) | pair, row0[seg_of_item], seg_len, slot],
                         axis=1)
        xcd_cus = _xcd_cus(device)
        all_items = self._xcd_schedule(items, cost, seg_of_item, item_start, xcd_cus)
        # The split kernel's schedule: segments of 1 .. SPLIT_MAX_ROWS rows as
        # sets, tile pairs for the longer ones.
        short = (flat >= 1) & (flat <= self.SPLIT_MAX_ROWS)
        if gram_dims is not None:
            k_op = np.asarray(gram_dims, dtype=np.int64).reshape(self.E, 2)
        else:
            k_op = np.repeat(weights[:, None] / 2.0, 2, axis=1)
        set_items = self._split_schedule(np.nonzero(short)[0], flat, row0, group,
                                         item_start[:-1], k_op)
        long_seg = ~short[seg_of_item]
        if long_seg.any():
            sub_counts = np.where(short, 0, npairs)
            sub_start = np.concatenate([[0], np.cumsum(sub_counts)])
            long_items = self._xcd_schedule(items[long_seg], cost[long_seg],
                                            seg_of_item[long_seg], sub_start, xcd_cus)
        else:
            long_items = np.zeros((0, 4), dtype=np.int64)
        self.n_sets = int(short.sum())
        self.max_steps = int(((flat + _STEP_ROWS - 1) // _STEP_ROWS).sum())
        # One int32 buffer: row0 [S] | len [S] | group [S] | rows [E] |
        # item_start [S + 1] | tile-pair items of every segment | tile-pair
        # items of the long segments | split items.
        parts = [row0, flat, group, self.rows, item_start, all_items.reshape(-1),
                 long_items.reshape(-1), set_items.reshape(-1)]
        buf = device_table(np.concatenate(parts), np.int32, device)
        offs = np.cumsum([0] + [len(p) for p in parts])
        (self.seg_row0, self.seg_len, self.seg_group, self.rows_dev, self.item_start,
         self.items, self.long_items, self.set_items) = [buf[offs[i]:offs[i + 1]]
                                                         for i in range(len(parts))]
        self.n_launch_items = len(all_items)
        self.n_long_items = len(long_items)
        self.n_set_items = len(set_items)
        self._buf = buf
        self.device = torch.device(device)


def _ptr_table(tensors, device) -> torch.Tensor:
    return pointer_table(tensors, device)


def _check_grouped(A_list, G_list, layout: SegmentLayout, *, same_shape: bool):
    if len(A_list) != layout.E or len(G_list) != layout.E:
        raise ConfigurationError("one A and one G per problem of the layout are required")
    if layout.E == 0:
        raise ConfigurationError("a grouped call needs at least one problem")
    din, dout, dtype = A_list[0].shape[-1], G_list[0].shape[-1], A_list[0].dtype
    for e, (A, G) in enumerate(zip(A_list, G_list)):
        if A.dim() != 2 or G.dim() != 2 or A.shape[0] != G.shape[0]:
            raise ConfigurationError("grouped operands must be A_e [rows, din], G_e [rows, dout]")
        if A.dtype != dtype or G.dtype != dtype:
            raise ConfigurationError("grouped problems must share a dtype")
        if same_shape and (A.shape[1] != din or G.shape[1] != dout):
            raise ConfigurationError("grouped problems must share din and dout")
        if A.shape[0] != int(layout.rows[e]):
            raise ConfigurationError(
                f"problem {e} has {A.shape[0]} rows, its segments {int(layout.rows[e])}")
        if not (A.is_contiguous() and G.is_contiguous()):
            raise ConfigurationError("grouped operands must be contiguous")
    return din, dout, dtype


def grouped_gram_sqnorms(A_list, G_list, layout: SegmentLayout, *, return_error: bool = False):
    """``||G_v^T A_v||^2`` for every segment v of the layout: float64 [E, K]
    (with ``return_error``, ``(seg_sq, seg_err)``: ``seg_err`` bounds the
    rounding error as in :func:`gram_sqnorms`).

    Problems may differ in din / dout (at most 64 problems per call)."""
    dev = nat.require_device(*A_list, *G_list)
    _, _, dtype = _check_grouped(A_list, G_list, layout, same_shape=False)
    if layout.E > SegmentLayout.MAX_GRAM_PROBLEMS:
        raise ConfigurationError("at most 64 problems per grouped Gram call")
    dims = (ctypes.c_int * (2 * layout.E))(
        *[v for A, G in zip(A_list, G_list) for v in (A.shape[1], G.shape[1])])
    seg_sq = torch.empty((layout.E, layout.K), dtype=torch.float64, device=dev)
    seg_err = (torch.empty((layout.E, layout.K), dtype=torch.float64, device=dev)
               if return_error else None)
    # The grouped split kernel (bf16, widths that are multiples of 8) takes the
    # segments of up to SPLIT_MAX_ROWS rows; the tile-pair kernel the rest.
    widths = [w for A, G in zip(A_list, G_list) for w in (A.shape[1], G.shape[1])]
    split = (dtype == torch.bfloat16 and layout.n_set_items > 0
             and all(w % 8 == 0 for w in widths)
             and SegmentLayout.SPLIT_MAX_ROWS * max(widths) * 2 < (1 << 31))
    if split:
        items, n_items = layout.long_items, layout.n_long_items
        sets, n_set_items, n_sets = layout.set_items, layout.n_set_items, layout.n_sets
    else:
        items, n_items = layout.items, layout.n_launch_items
        sets, n_set_items, n_sets = None, 0, 0
    n_records = layout.n_items
    nbytes = nat.load().dpc_grouped_gram_workspace_bytes(n_records, n_sets)
    ws = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=dev)
    a_ptrs, g_ptrs = _ptr_table(A_list, dev), _ptr_table(G_list, dev)
    nat.call(
        "dpc_grouped_gram_sqnorms", nat.ptr(a_ptrs), nat.ptr(g_ptrs), dims, layout.E,
        nat.dtype_code(dtype), nat.ptr(items), n_items, layout.max_rows, nat.ptr(sets),
        n_set_items, n_sets, n_records, nat.ptr(layout.item_start), layout.S, nat.ptr(seg_sq),
        nat.ptr(seg_err), nat.ptr(ws), ws.numel(), nat.stream_handle(dev),
    )
    return (seg_sq, seg_err) if return_error else seg_sq


@dataclass
class GroupedNoise:
    """Noise of a grouped clipped sum: per-problem ``sigmas``; ``noise`` holds
    float32 draws per problem (mode INJECTED) or ``leaf_ids`` name each
    problem's Philox stream under ``seed`` (mode PHILOX)."""

    sigmas: list
    mode: int = nat.NOISE_PHILOX
    noise: list | None = None
    seed: int = 0
    leaf_ids: list | None = None


def grouped_clipped_sum(
    A_list,
    G_list,
    layout: SegmentLayout,
    seg_scale: torch.Tensor,
    *,
    normalize_by: float = 1.0,
    noise: GroupedNoise | None = None,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """``out[e] = sum_v seg_scale[v] G_v^T A_v`` over problem e's segments, with
    ``/ normalize_by`` and noise in the epilogue: [E, dout, din].

    ``seg_scale`` is float32 [E, K] (segment v = e * K + k); segments with
    scale 0 are never read.
    """
    dev = nat.require_device(*A_list, *G_list, seg_scale)
    din, dout, dtype = _check_grouped(A_list, G_list, layout, same_shape=True)
    if seg_scale.dtype != torch.float32 or tuple(seg_scale.shape) != (layout.E, layout.K):
        raise ConfigurationError("seg_scale must be float32 [E, K]")
    seg_scale = _contig(seg_scale)
    out_dtype = out_dtype or dtype
    E = layout.E
    out = torch.empty((E, dout, din), dtype=out_dtype, device=dev)
    steps = torch.empty(2 * max(layout.max_steps, 1), dtype=torch.int32, device=dev)
    step_start = torch.empty(E + 1, dtype=torch.int32, device=dev)
    stream = nat.stream_handle(dev)
    nat.call(
        "dpc_segment_plan", nat.ptr(layout.seg_row0), nat.ptr(layout.seg_len),
        nat.ptr(layout.seg_group), nat.ptr(seg_scale), layout.S, E, layout.max_steps,
        nat.ptr(steps), nat.ptr(step_start), stream,
    )
    spec = noise or GroupedNoise(sigmas=[0.0] * E, mode=nat.NOISE_NONE)
    if len(spec.sigmas) != E:
        raise ConfigurationError("one noise sigma per problem is required")
    active = any(s != 0.0 for s in spec.sigmas)
    mode = spec.mode if active else nat.NOISE_NONE
    noise_ptrs = None
    if mode == nat.NOISE_INJECTED:
        if spec.noise is None or len(spec.noise) != E:
            raise ConfigurationError("injected noise needs one float32 tensor per problem")
        for t in spec.noise:
            if t.dtype != torch.float32 or tuple(t.shape) != (dout, din) or not t.is_contiguous() \
                    or t.device != dev:
                raise ConfigurationError(f"injected noise must be float32 {(dout, din)} on the device")
        noise_ptrs = _ptr_table(spec.noise, dev)
    leaf_ids = spec.leaf_ids if spec.leaf_ids is not None else list(range(E))
    if len(leaf_ids) != E:
        raise ConfigurationError("one leaf id per problem is required")
    leaf_dev = device_table([v & 0xFFFFFFFF for v in leaf_ids], np.uint32, dev)
    sig_dev = device_table([float(v) for v in spec.sigmas], np.float32, dev)
    a_ptrs, g_ptrs = _ptr_table(A_list, dev), _ptr_table(G_list, dev)
    out_ptrs = _ptr_table([out[e] for e in range(E)], dev)
    nat.call(
        "dpc_grouped_clipped_sum", nat.ptr(a_ptrs), nat.ptr(g_ptrs), nat.ptr(layout.rows_dev),
        layout.max_rows, E, din, dout, nat.dtype_code(dtype), nat.ptr(steps),
        nat.ptr(step_start), nat.ptr(seg_scale), float(normalize_by), mode, nat.ptr(noise_ptrs),
        spec.seed & ((1 << 64) - 1), nat.ptr(leaf_dev), nat.ptr(sig_dev),
        nat.dtype_code(out_dtype), nat.ptr(out_ptrs), stream,
    )
    return out


NARROW_MAX = 32  # widest narrow side of dpc_per_example_grads


def per_example_grads(A: torch.Tensor, G: torch.Tensor, *,
                      out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Per-example weight gradients ``G_i^T A_i`` of a linear layer whose din or
    dout is at most 32: [B, dout, din] in ``out_dtype`` (default: the input
    dtype), summed in float32."""
    dev = nat.require_device(A, G)
    if A.dim() != 3 or G.dim() != 3 or A.shape[:2] != G.shape[:2] or A.dtype != G.dtype:
        raise ConfigurationError("expected A [B, T, din], G [B, T, dout] of one dtype")
    B, T, din = A.shape
    dout = G.shape[2]
    if min(din, dout) > NARROW_MAX:
        raise ConfigurationError(f"per_example_grads needs din or dout <= {NARROW_MAX}")
    out_dtype = out_dtype or A.dtype
    out = torch.empty((B, dout, din), dtype=out_dtype, device=dev)
    if B == 0:
        return out
    # The kernel reads rows with aligned vector loads.
    A = A.contiguous() if (A.is_contiguous() and A.data_ptr() % 16 == 0) else A.clone(
        memory_format=torch.contiguous_format)
    G = G.contiguous() if (G.is_contiguous() and G.data_ptr() % 16 == 0) else G.clone(
        memory_format=torch.contiguous_format)
    ws_bytes = nat.load().dpc_per_example_grads_workspace_bytes(B, T, din, dout)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    nat.call("dpc_per_example_grads", nat.ptr(A), nat.ptr(G), B, T, din, dout,
             nat.dtype_code(A.dtype), nat.ptr(out), nat.dtype_code(out_dtype), nat.ptr(ws),
             ws_bytes, nat.stream_handle(dev))
    return out


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous and 16-byte aligned (the kernels read rows with aligned
    vector loads)."""
    if t.is_contiguous() and t.data_ptr() % 16 == 0:
        return t
    return t.clone(memory_format=torch.contiguous_format)


def per_example_grads_grouped(A_list, G_list, *,
                              out_dtype: torch.dtype | None = None) -> list[torch.Tensor]:
    """``per_example_grads`` of several layers that share the batch and token
    count (``dpc_per_example_grads_grouped``: the eligible bfloat16 layers
    share MFMA launches).  Returns one [B, dout, din] tensor per layer."""
    if len(A_list) != len(G_list) or not A_list:
        raise ConfigurationError("expected matching, non-empty lists of A and G")
    dev = nat.require_device(*A_list, *G_list)
    dtype = A_list[0].dtype
    B, T = A_list[0].shape[:2]
    for A, G in zip(A_list, G_list):
        if A.dim() != 3 or G.dim() != 3 or A.shape[:2] != (B, T) or G.shape[:2] != (B, T):
            raise ConfigurationError("expected A [B, T, din], G [B, T, dout] with one B and T")
        if A.dtype != dtype or G.dtype != dtype:
            raise ConfigurationError("the layers' operands must share one dtype")
        if min(A.shape[2], G.shape[2]) > NARROW_MAX:
            raise ConfigurationError(f"per_example_grads needs din or dout <= {NARROW_MAX}")
    out_dtype = out_dtype or dtype
    n = len(A_list)
    dins = [A.shape[2] for A in A_list]
    douts = [G.shape[2] for G in G_list]
    outs = [torch.empty((B, o, i), dtype=out_dtype, device=dev) for i, o in zip(dins, douts)]
    if B == 0:
        return outs
    # A tensor passed for several layers stays one buffer (layers that share
    # their wide operand share the kernel's pass over it).
    seen = {}

    def once(t):
        if id(t) not in seen:
            seen[id(t)] = _aligned(t)
        return seen[id(t)]

    As = [once(A) for A in A_list]
    Gs = [once(G) for G in G_list]
    c_din = (ctypes.c_int * n)(*dins)
    c_dout = (ctypes.c_int * n)(*douts)
    ws_bytes = nat.load().dpc_per_example_grads_grouped_workspace_bytes(
        n, c_din, c_dout, B, T, nat.dtype_code(dtype))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    nat.call("dpc_per_example_grads_grouped", n, (ctypes.c_void_p * n)(*[t.data_ptr() for t in As]),
             (ctypes.c_void_p * n)(*[t.data_ptr() for t in Gs]),
             (ctypes.c_void_p * n)(*[t.data_ptr() for t in outs]), c_din, c_dout, B, T,
             nat.dtype_code(dtype), nat.dtype_code(out_dtype), nat.ptr(ws), ws_bytes,
             nat.stream_handle(dev))
    return outs


def leaf_view(t: torch.Tensor) -> tuple[int, int]:
    """The [rows, cols] view of a leaf for the device noise stream."""
    if t.dim() == 0:
        return 1, 1
    rows = t.shape[0]
    return rows, (t.numel() // rows if rows else 0)


def add_noise(
    x: torch.Tensor,
    sigma: float,
    *,
    mode: int = nat.NOISE_PHILOX,
    noise: torch.Tensor | None = None,
    seed: int = 0,
    leaf_id: int = 0,
    compute_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Out-of-place ``to_dtype(to_cd(to_cd(x) + to_cd(sigma * z)))`` with
    ``cd = compute_dtype`` (float32: ``to_dtype(float(x) + float32(sigma) *
    z)``).  Injected ``noise`` is a ``compute_dtype`` tensor shaped like
    ``x``.  float32 / bfloat16 leaves with a float32 compute dtype take
    ``dpc_add_noise``, every other combination ``dpc_add_noise_ex``."""
    dev = nat.require_device(x, noise)
    x = _contig(x)
    y = torch.empty_like(x)
    rows, cols = leaf_view(x)
    if mode == nat.NOISE_INJECTED and sigma != 0.0:
        if noise is None or noise.dtype != compute_dtype or noise.shape != x.shape:
            raise ConfigurationError(
                f"injected noise must be {compute_dtype} shaped like the leaf")
        noise = _contig(noise)
    seed &= (1 << 64) - 1
    if compute_dtype == torch.float32 and x.dtype in (torch.float32, torch.bfloat16):
        nat.call(
            "dpc_add_noise", nat.ptr(x), nat.ptr(y), rows, cols, nat.dtype_code(x.dtype),
            float(sigma), mode, nat.ptr(noise), seed, leaf_id & 0xFFFFFFFF,
            nat.stream_handle(dev),
        )
    else:
        nat.call(
            "dpc_add_noise_ex", nat.ptr(x), nat.ptr(y), rows, cols,
            nat.dtype_code(x.dtype, wide=True), nat.dtype_code(compute_dtype, wide=True),
            float(sigma), mode, nat.ptr(noise), seed, leaf_id & 0xFFFFFFFF,
            nat.stream_handle(dev),
        )
    return y


def sanitize_columns(x: torch.Tensor) -> torch.Tensor:
    """``x`` [n, T, d] with every column (over T) of each matrix that holds a
    non-finite value set to zero (``dpc_sanitize_columns``)."""
    dev = nat.require_device(x)
    if x.dim() != 3:
        raise ConfigurationError("expected x [n, T, d]")
    x = _contig(x)
    out = torch.empty_like(x)
    nat.call("dpc_sanitize_columns", nat.ptr(x), nat.ptr(out), x.shape[0], x.shape[1],
             x.shape[2], nat.dtype_code(x.dtype, wide=True), nat.stream_handle(dev))
    return out


def add_noise_leaves(xs, sigmas, *, seed: int, leaf_ids, inplace: bool = False
                     ) -> list[torch.Tensor]:
    """``add_noise`` (Philox stream) of several leaves of one dtype in as few
    launches as possible (``dpc_add_noise_leaves``); each result equals
    ``add_noise(x, sigma, seed=seed, leaf_id=leaf_id)``.  With ``inplace``
    the (contiguous) leaves themselves receive the noise."""
    if not (len(xs) == len(sigmas) == len(leaf_ids)) or not xs:
        raise ConfigurationError("expected matching, non-empty lists of leaves, sigmas and ids")
    dev = nat.require_device(*xs)
    dtype = xs[0].dtype
    if any(x.dtype != dtype for x in xs):
        raise ConfigurationError("the leaves must share one dtype")
    if inplace and not all(x.is_contiguous() for x in xs):
        raise ConfigurationError("in-place noise needs contiguous leaves")
    xs = [_contig(x) for x in xs]
    ys = xs if inplace else [torch.empty_like(x) for x in xs]
    n = len(xs)
    views = [leaf_view(x) for x in xs]
    nat.call("dpc_add_noise_leaves", n, (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs]),
             (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]),
             (ctypes.c_int64 * n)(*[r for r, _ in views]),
             (ctypes.c_int64 * n)(*[c for _, c in views]),
             (ctypes.c_double * n)(*[float(v) for v in sigmas]),
             (ctypes.c_uint32 * n)(*[i & 0xFFFFFFFF for i in leaf_ids]),
             nat.dtype_code(dtype), seed & ((1 << 64) - 1), nat.stream_handle(dev))
    return ys


def philox4x32_10(counter: tuple[int, int, int, int], key: tuple[int, int], n: int,
                  device: torch.device | str = "cuda") -> torch.Tensor:
    """``n`` Philox4x32-10 blocks for counters ``(c0 + j, c1, c2, c3)``: int64 [n, 4]."""
    device = torch.device(device)
    out = torch.empty((max(n, 1), 4), dtype=torch.int32, device=device)
    nat.call(
        "dpc_philox4x32_10", *[c & 0xFFFFFFFF for c in counter], *[k & 0xFFFFFFFF for k in key],
        n, nat.ptr(out), nat.stream_handle(device),
    )
    return out[:n].to(torch.int64) & 0xFFFFFFFF


__all__ = [
    "ClipFactorGroups",
    "ClipFactors",
    "clip_factors_groups",
    "gram_clip_factors",
    "sanitize_columns",
    "GroupedNoise",
    "NoiseSpec",
    "SegmentLayout",
    "add_noise",
    "clip_factors",
    "clipped_sum",
    "clipped_sum_multi",
    "gram_sqnorms_multi",
    "flat_sqnorms",
    "gram_sqnorms",
    "grouped_clipped_sum",
    "grouped_gram_sqnorms",
    "leaf_view",
    "per_example_grads",
    "philox4x32_10",
]
