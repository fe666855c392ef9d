"""Per-example clipping engine (HIP kernels behind the reference's API)."""

from opake_amd.clipping._ghost import GhostClipAux, ghost_clip_sum, ghost_sqnorms, guard_for_linear

__all__ = ["GhostClipAux", "ghost_clip_sum", "ghost_sqnorms", "guard_for_linear"]
