"""Per-group Gaussian noise allocation.

``per_group_noise_stddev`` follows the reference
(``packages/opake-engine/src/opake/api/engine/noise_allocation.py:44-110``):
``sigma_k = nm * sqrt(C_k * sum_j C_j)``; ``nm == 0`` gives exact zeros even
for infinite bounds.
"""

from __future__ import annotations

import math

from opake_amd.exceptions import ConfigurationError, InputTypeError
from opake_amd.types import PerGroup

PAIRED_FIRST_STREAM_FOLD = "opake.paired.first"
PAIRED_SECOND_STREAM_FOLD = "opake.paired.second"


def per_group_noise_stddev(max_norm: PerGroup, noise_multiplier: float) -> PerGroup:
    if not isinstance(max_norm, PerGroup):
        raise InputTypeError(
            "per_group_noise_stddev requires a PerGroup max_norm, "
            f"got {type(max_norm).__name__}."
        )
    if noise_multiplier < 0:
        raise ConfigurationError(
            f"noise_multiplier must be non-negative, got {noise_multiplier}"
        )
    for name, value in max_norm.values.items():
        if value < 0:
            raise ConfigurationError(
                f"per-group bounds must be non-negative, got {value} for group '{name}'."
            )
    if noise_multiplier == 0.0:
        return PerGroup(max_norm.groups, dict.fromkeys(max_norm.values, 0.0))
    total = sum(max_norm.values.values())
    return PerGroup(
        max_norm.groups,
        {k: noise_multiplier * math.sqrt(c * total) for k, c in max_norm.values.items()},
    )


__all__ = [
    "PAIRED_FIRST_STREAM_FOLD",
    "PAIRED_SECOND_STREAM_FOLD",
    "per_group_noise_stddev",
]
