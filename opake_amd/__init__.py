"""MI355X-native DP-SGD per-example clip -> sum -> Gaussian-noise step.

A drop-in for the hot path behind JetBrains-Research/opake's
``opake.dpsgd.clipping`` / ``opake.api.engine.clipping`` (``ClippedPytree``)
and ``opake.dpsgd.noise`` (``NoisedPytree``): the same functional API and
types, with the work done by hand-written HIP kernels for gfx950 behind the C
ABI in ``include/opake_amd.h``.
"""

import os as _os

# Kernel arguments in device memory: the first waves of a launch read them
# without a round trip to host memory (4-5 us less per config-2 step, two
# launches).  HIP reads this when its runtime starts, so it takes effect
# only if nothing in the process has used the GPU yet; a value the caller
# set is kept.
_os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "1")

from opake_amd import exceptions, random, types  # noqa: E402
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
