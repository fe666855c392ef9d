"""Tensor-level wrappers of the native kernels.

Each function validates shapes on the host, allocates outputs and scratch with
torch on the inputs' device, and enqueues the kernels on the current stream.
None of them synchronises the host.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from opake_amd import _native as nat
from opake_amd.exceptions import ConfigurationError


def _contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def gram_sqnorms(
    A: torch.Tensor,
    G: torch.Tensor,
    *,
    with_bias: bool = False,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``out[i] (+)= ||G_i^T A_i||_F^2 (+ ||sum_t G_i[t]||^2)`` in float64.

    ``A``: [B, T, din], ``G``: [B, T, dout], same dtype (bf16 or fp32).  When
    ``out`` is given the layer's contribution is added to it.
    """
    dev = nat.require_device(A, G, out)
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
    if out is None:
        out = torch.empty(B, dtype=torch.float64, device=dev)
    elif out.dtype != torch.float64 or out.shape != (B,):
        raise ConfigurationError("out must be float64 [B]")
    if B == 0:
        return out
    ws_bytes = nat.load().dpc_gram_workspace_bytes(B, T)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    nat.call(
        "dpc_gram_sqnorms", nat.ptr(A), nat.ptr(G), B, T, din, dout, nat.dtype_code(A.dtype),
        int(with_bias), int(accumulate), nat.ptr(out), nat.ptr(ws), ws_bytes,
        nat.stream_handle(dev),
    )
    return out


def flat_sqnorms(
    a: torch.Tensor,
    g: torch.Tensor,
    *,
    with_bias: bool = False,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``out[i] (+)= ||a_i||^2 ||g_i||^2 (+ ||g_i||^2)`` for flat inputs [B, d]."""
    dev = nat.require_device(a, g, out)
    if a.dim() != 2 or g.dim() != 2 or a.shape[0] != g.shape[0] or a.dtype != g.dtype:
        raise ConfigurationError("expected a [B, din] and g [B, dout] of one dtype")
    B, din = a.shape
    dout = g.shape[1]
    accumulate = out is not None
    if out is None:
        out = torch.empty(B, dtype=torch.float64, device=dev)
    if B == 0:
        return out
    a, g = _contig(a), _contig(g)
    nat.call(
        "dpc_flat_sqnorms", nat.ptr(a), nat.ptr(g), B, din, dout, nat.dtype_code(a.dtype),
        int(with_bias), int(accumulate), nat.ptr(out), nat.stream_handle(dev),
    )
    return out


@dataclass
class ClipFactors:
    """Outputs of :func:`clip_factors` (all on device, nothing synchronised)."""

    scale: torch.Tensor  # float32 [n_guards, B]
    norms: torch.Tensor  # float32 [B]
    nclipped: torch.Tensor  # int32 [1]
    plan: torch.Tensor  # uint8 plan bytes (active example list of guard 0)


def clip_factors(
    sqnorm: torch.Tensor,
    clipping_norm: float,
    guards: list[tuple[float, float]],
    *,
    kind: int = nat.SCALE_FIXED,
    gamma: float = 0.0,
    count_threshold: float,
) -> ClipFactors:
    """Guarded clip factors for each ``(rel, abs)`` guard, per example."""
    dev = nat.require_device(sqnorm)
    if sqnorm.dtype != torch.float64 or sqnorm.dim() != 1:
        raise ConfigurationError("sqnorm must be a float64 vector")
    if not 1 <= len(guards) <= 4:
        raise ConfigurationError("between 1 and 4 guards are supported")
    B = sqnorm.shape[0]
    n = len(guards)
    rel = (ctypes.c_double * n)(*[g[0] for g in guards])
    abs_ = (ctypes.c_double * n)(*[g[1] for g in guards])
    scale = torch.empty((n, B), dtype=torch.float32, device=dev)
    norms = torch.empty(B, dtype=torch.float32, device=dev)
    nclipped = torch.empty(1, dtype=torch.int32, device=dev)
    plan = torch.empty(nat.load().dpc_clip_plan_bytes(B), dtype=torch.uint8, device=dev)
    nat.call(
        "dpc_clip_factors", nat.ptr(_contig(sqnorm)), B, float(clipping_norm), kind, float(gamma),
        rel, abs_, n, float(count_threshold), nat.ptr(scale), nat.ptr(norms), nat.ptr(nclipped),
        nat.ptr(plan), nat.stream_handle(dev),
    )
    return ClipFactors(scale=scale, norms=norms, nclipped=nclipped, plan=plan)


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
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if with_bias else None
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
        int(with_bias), nat.ptr(bias_out), nat.ptr(ws), ws_bytes if with_bias else 0,
        nat.stream_handle(dev),
    )
    return out, bias_out


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
) -> torch.Tensor:
    """Out-of-place ``to_dtype(float(x) + float32(sigma) * z)``."""
    dev = nat.require_device(x, noise)
    x = _contig(x)
    y = torch.empty_like(x)
    rows, cols = leaf_view(x)
    if mode == nat.NOISE_INJECTED and sigma != 0.0:
        if noise is None or noise.dtype != torch.float32 or noise.shape != x.shape:
            raise ConfigurationError("injected noise must be float32 shaped like the leaf")
        noise = _contig(noise)
    nat.call(
        "dpc_add_noise", nat.ptr(x), nat.ptr(y), rows, cols, nat.dtype_code(x.dtype),
        float(sigma), mode, nat.ptr(noise), seed & ((1 << 64) - 1), leaf_id & 0xFFFFFFFF,
        nat.stream_handle(dev),
    )
    return y


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
    "ClipFactors",
    "NoiseSpec",
    "add_noise",
    "clip_factors",
    "clipped_sum",
    "flat_sqnorms",
    "gram_sqnorms",
    "leaf_view",
    "philox4x32_10",
]
