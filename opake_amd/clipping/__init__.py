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
from opake_amd.clipping._model import (
    DirectCapture,
    GhostGradAux,
    LinearCapture,
    auto_ghost_clipped_grad,
    ghost_capture,
    ghost_clip_captured,
    ghost_clipped_grad,
)
from opake_amd.clipping._leaves import (
    LeafClipResult,
    fused_stream_clip_and_sum,
    get_fused_clip_backend,
    leaves_clip_sum,
    make_fused_backend,
    register_fused_clip_backend,
)
from opake_amd.clipping._pytree_clip import ClipPytreeAux, auto_scale_pytree, clip_pytree
from opake_amd.clipping._graph import GraphedGhostClip

__all__ = [
    "AutoClipState",
    "ClipPytreeAux",
    "ClippedFunAux",
    "ClippedGradAux",
    "DirectCapture",
    "ClippingStats",
    "FixedClipState",
    "GhostClipAux",
    "GhostGradAux",
    "GraphedGhostClip",
    "LeafClipResult",
    "LinearCapture",
    "auto_clipped_grad",
    "auto_ghost_clipped_grad",
    "auto_scale_pytree",
    "clip_pytree",
    "clipped_fun",
    "clipped_grad",
    "fused_stream_clip_and_sum",
    "get_fused_clip_backend",
    "ghost_capture",
    "ghost_clip_captured",
    "ghost_clip_sum",
    "ghost_clipped_grad",
    "ghost_sqnorms",
    "guard_for_linear",
    "leaves_clip_sum",
    "make_fused_backend",
    "register_fused_clip_backend",
]
