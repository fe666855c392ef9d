"""MI355X-native DP-SGD per-example clip -> sum -> Gaussian-noise step.

A drop-in for the hot path behind JetBrains-Research/opake's
``opake.dpsgd.clipping`` / ``opake.api.engine.clipping`` (``ClippedPytree``)
and ``opake.dpsgd.noise`` (``NoisedPytree``): the same functional API and
types, with the work done by hand-written HIP kernels for gfx950 behind the C
ABI in ``include/opake_amd.h``.
"""

from opake_amd import exceptions, random, types
from opake_amd.random import RngKey, fold_in, generator_from_key, key, split
from opake_amd.types import (
    ClippedPytree,
    NoisedPytree,
    PerGroup,
    SecondMomentClippingOutput,
    SecondMomentNoiseOutput,
    clipped,
    noised,
)

__version__ = "0.1.0"

__all__ = [
    "ClippedPytree",
    "NoisedPytree",
    "PerGroup",
    "RngKey",
    "SecondMomentClippingOutput",
    "SecondMomentNoiseOutput",
    "clipped",
    "exceptions",
    "fold_in",
    "generator_from_key",
    "key",
    "noised",
    "random",
    "split",
    "types",
]
