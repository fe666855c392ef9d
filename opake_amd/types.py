"""DP wrapper types that connect clipping, noise and the optimizer.

Same interface and semantics as the reference's
``packages/opake-engine/src/opake/api/engine/types.py:71-477``:

* ``PerGroup`` (``types.py:71-163``): leaf-path -> group mapping plus per-group
  values; ``effective = sqrt(sum v^2)``; scalar and element-wise arithmetic.
* ``ClippedPytree`` (``:259-393``): a pytree with a public ``max_norm``.  Only
  public-scalar ``*``, ``/`` and negation keep the DP interpretation; ``+``,
  ``-`` and ``**`` raise ``InputTypeError``.
* ``NoisedPytree`` (``:396-413``): adds the realised ``noise_stddev``.
* ``clipped()`` / ``noised()`` factories (``:465-477``).
"""

from __future__ import annotations

import math
from abc import ABC
from dataclasses import dataclass, replace
from numbers import Real
from types import MappingProxyType
from typing import Any, Literal, Mapping, NamedTuple

import torch

from opake_amd.exceptions import ConfigurationError, InputTypeError
from opake_amd.pytree import ParamPath, param_path, tree_map


@dataclass(frozen=True)
class PerGroup:
    """Per-group scalar values with a pre-resolved leaf-path -> group map."""

    groups: Mapping[Any, str]
    values: Mapping[str, float]

    def __post_init__(self) -> None:
        normalized = {param_path(k): g for k, g in self.groups.items()}
        object.__setattr__(self, "groups", MappingProxyType(normalized))
        object.__setattr__(self, "values", MappingProxyType(dict(self.values)))

    @property
    def effective(self) -> float:
        return math.sqrt(sum(v * v for v in self.values.values()))

    @property
    def num_groups(self) -> int:
        return len(self.values)

    def _map(self, fn) -> "PerGroup":
        return PerGroup(self.groups, {k: fn(k, v) for k, v in self.values.items()})

    def __rmul__(self, scalar: float) -> "PerGroup":
        return self._map(lambda _k, v: scalar * v)

    def __mul__(self, other) -> "PerGroup":
        if isinstance(other, PerGroup):
            if dict(other.groups) != dict(self.groups):
                raise ConfigurationError(
                    "PerGroup × PerGroup requires identical group mappings; got "
                    f"groups with {len(self.groups)} vs {len(other.groups)} "
                    "parameter assignments."
                )
            if set(other.values) != set(self.values):
                raise ConfigurationError(
                    "PerGroup × PerGroup requires identical group sets; got "
                    f"{sorted(self.values)} vs {sorted(other.values)}."
                )
            return self._map(lambda k, v: v * other.values[k])
        return self._map(lambda _k, v: v * other)

    def __truediv__(self, scalar: float) -> "PerGroup":
        return self._map(lambda _k, v: v / scalar)

    def for_path(self, path) -> float:
        return self.values[self.groups[param_path(path)]]


class ClipState(ABC):  # noqa: B024 - marker base, as in the reference
    """Base of clipping states (reference ``types.py:170-179``)."""


class NoiseState(ABC):
    """Base of noise states (reference ``types.py:182-198``)."""

    _step_counter: int
    _rng_key: Any


MaxNorm = Any
NoiseStddev = Any


def _public_scalar(scalar: Any, *, op: str) -> float:
    if isinstance(scalar, bool) or not isinstance(scalar, Real):
        raise InputTypeError(
            f"{op} only supports public real-number scalars. Operate on `.pytree` "
            "and reconstruct the clipped value with an explicit max_norm when the "
            "clipped interpretation is unclear."
        )
    return float(scalar)


def _unsupported(op: str) -> str:
    return (
        f"ClippedPytree {op} does not preserve DP max_norm semantics automatically. "
        "Operate on `.pytree` and reconstruct the clipped value with an explicit "
        "max_norm."
    )


def _tensor_method(pytree: Any, method: str, *args, **kwargs) -> Any:
    return tree_map(
        lambda x: getattr(x, method)(*args, **kwargs) if isinstance(x, torch.Tensor) else x,
        pytree,
    )


@dataclass(frozen=True)
class ClippedPytree:
    """A pytree whose per-record contribution has L2 norm at most ``max_norm``."""

    pytree: Any
    max_norm: MaxNorm

    @property
    def sensitivity(self) -> float:
        eff = getattr(self.max_norm, "effective", None)
        return float(eff) if eff is not None else float(self.max_norm)

    def noise_stddev_for(
        self,
        *,
        noise_multiplier: float,
        allocation: Literal["isotropic", "optimal"] = "optimal",
    ):
        if noise_multiplier < 0:
            raise ConfigurationError(
                f"noise_multiplier must be non-negative, got {noise_multiplier}"
            )
        if allocation not in ("isotropic", "optimal"):
            raise ConfigurationError(
                f"allocation must be 'isotropic' or 'optimal', got {allocation!r}."
            )
        if isinstance(self.max_norm, PerGroup):
            if allocation == "isotropic":
                return noise_multiplier * self.max_norm.effective
            from opake_amd.noise_allocation import per_group_noise_stddev

            return per_group_noise_stddev(self.max_norm, noise_multiplier)
        return noise_multiplier * float(self.max_norm)

    def _scaled(self, factor: float):
        return replace(
            self,
            pytree=tree_map(
                lambda x: x * factor if isinstance(x, torch.Tensor) else x, self.pytree
            ),
            max_norm=abs(factor) * self.max_norm,
        )

    def __mul__(self, s):
        return self._scaled(_public_scalar(s, op="ClippedPytree *"))

    def __rmul__(self, s):
        return self._scaled(_public_scalar(s, op="* ClippedPytree"))

    def __truediv__(self, s):
        f = _public_scalar(s, op="ClippedPytree /")
        if f == 0.0:
            raise ZeroDivisionError("ClippedPytree division by zero")
        return self._scaled(1.0 / f)

    def __rtruediv__(self, s):
        raise InputTypeError(_unsupported("reverse division"))

    def __neg__(self):
        return self._scaled(-1.0)

    def __add__(self, o):
        raise InputTypeError(_unsupported("addition"))

    def __radd__(self, o):
        raise InputTypeError(_unsupported("addition"))

    def __sub__(self, o):
        raise InputTypeError(_unsupported("subtraction"))

    def __rsub__(self, o):
        raise InputTypeError(_unsupported("subtraction"))

    def __pow__(self, o):
        raise InputTypeError(_unsupported("power"))

    def clone(self):
        return replace(self, pytree=_tensor_method(self.pytree, "clone"))

    def detach(self):
        return replace(self, pytree=_tensor_method(self.pytree, "detach"))

    def to(self, *args, **kwargs):
        return replace(self, pytree=_tensor_method(self.pytree, "to", *args, **kwargs))


@dataclass(frozen=True)
class NoisedPytree(ClippedPytree):
    """A privatised pytree with the realised per-step ``noise_stddev``."""

    noise_stddev: NoiseStddev = None

    def _scaled(self, factor: float):
        return replace(
            self,
            pytree=tree_map(
                lambda x: x * factor if isinstance(x, torch.Tensor) else x, self.pytree
            ),
            max_norm=abs(factor) * self.max_norm,
            noise_stddev=None if self.noise_stddev is None else abs(factor) * self.noise_stddev,
        )


class SecondMomentClippingOutput(NamedTuple):
    """Pre-noise paired stream: ``sum_i g_i`` and ``sum_i g_i^2``."""

    grads: ClippedPytree
    squared_grads: ClippedPytree


class SecondMomentNoiseOutput(NamedTuple):
    noisy_grads: NoisedPytree
    noisy_squared_grads: NoisedPytree


def clipped(pytree: Any, *, max_norm: MaxNorm) -> ClippedPytree:
    return ClippedPytree(pytree=pytree, max_norm=max_norm)


def noised(pytree: Any, *, max_norm: MaxNorm, noise_stddev: NoiseStddev) -> NoisedPytree:
    return NoisedPytree(pytree=pytree, max_norm=max_norm, noise_stddev=noise_stddev)


__all__ = [
    "ClipState",
    "ClippedPytree",
    "MaxNorm",
    "NoiseState",
    "NoiseStddev",
    "NoisedPytree",
    "ParamPath",
    "PerGroup",
    "SecondMomentClippingOutput",
    "SecondMomentNoiseOutput",
    "clipped",
    "noised",
]
