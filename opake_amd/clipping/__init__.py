"""Per-example clipping engine (HIP kernels behind the reference's API)."""

from opake_amd.clipping._clipped_fun import (
    AutoClipState,
    ClippedFunAux,
    ClippedGradAux,
    ClippingStats,
    FixedClipState,
    auto_clipped_grad,
    clipped_fun,
    clipped_grad,
)
from opake_amd.clipping._ghost import GhostClipAux, ghost_clip_sum, ghost_sqnorms, guard_for_linear
from opake_amd.clipping._model import GhostGradAux, ghost_clipped_grad
from opake_amd.clipping._leaves import (
    fused_stream_clip_and_sum,
    get_fused_clip_backend,
    leaves_clip_sum,
    make_fused_backend,
    register_fused_clip_backend,
)

__all__ = [
    "AutoClipState",
    "ClippedFunAux",
    "ClippedGradAux",
    "ClippingStats",
    "FixedClipState",
    "GhostClipAux",
    "GhostGradAux",
    "auto_clipped_grad",
    "clipped_fun",
    "clipped_grad",
    "fused_stream_clip_and_sum",
    "get_fused_clip_backend",
    "ghost_clip_sum",
    "ghost_clipped_grad",
    "ghost_sqnorms",
    "guard_for_linear",
    "leaves_clip_sum",
    "make_fused_backend",
    "register_fused_clip_backend",
]
