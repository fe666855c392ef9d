"""Gaussian noise for clipped DP queries.

Same call sites and types as the reference's ``gaussian_noise``
(packages/opake-dpsgd/src/opake/api/dpsgd/noise/_gaussian.py:125-345):
``gaussian_noise(noise_multiplier=, key=, compute_dtype=)`` returns
``(noise_fn, state)``; ``noise_fn(ClippedPytree, state)`` returns
``(NoisedPytree, state')`` with ``noise_stddev = nm * max_norm`` (per-group:
``nm * sqrt(C_k * sum C)``); a ``SecondMomentClippingOutput`` gets two streams.
Step ``t`` draws from ``fold_in(key, "opake.dpsgd.gaussian", t)``.

The addition runs in a HIP kernel (``dpc_add_noise``) on the leaf's device.
``stream`` selects where the standard normals come from:

* ``"reference"`` (default): the reference's own stream -- a CPU
  ``torch.Generator`` seeded from the step key, ``torch.randn`` per leaf in
  flatten order -- copied to the device and added there.  Results are
  bit-identical to the reference for the same inputs.
* ``"device"``: a Philox4x32-10 / Box-Muller stream generated in the kernel
  from the same step key and the leaf's flatten index.  It is a *different*
  stream with the same distribution; it does not depend on which device or
  how many devices run it.  No host work or copy, so it is the fast path.

Supported: float16 / bfloat16 / float32 / float64 leaves on a ROCm device and
each of those compute dtypes: the draw (``torch.randn(dtype=compute_dtype)``
in the reference stream, the Philox normal rounded to it in the device
stream), the scaling and the addition happen in ``compute_dtype`` and the
result is cast back to the leaf dtype, as ``_gaussian.py:188-204`` does.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Any

import torch
from torch.autograd.profiler import record_function

from opake_amd import _native as nat
from opake_amd import ops
from opake_amd.exceptions import ConfigurationError, InputTypeError, OperationError
from opake_amd.noise_allocation import (
    PAIRED_FIRST_STREAM_FOLD,
    PAIRED_SECOND_STREAM_FOLD,
    per_group_noise_stddev,
)
from opake_amd.pytree import tree_flatten_with_paths, tree_unflatten
from opake_amd.random import RngKey, fold_in, generator_from_key
from opake_amd.types import (
    ClippedPytree,
    NoisedPytree,
    NoiseState,
    PerGroup,
    SecondMomentClippingOutput,
    SecondMomentNoiseOutput,
)

GAUSSIAN_STREAM_FOLD = "opake.dpsgd.gaussian"
STREAMS = ("reference", "device")
_SUPPORTED_COMPUTE = frozenset({torch.float16, torch.bfloat16, torch.float32, torch.float64})


@dataclasses.dataclass(frozen=True)
class GaussianNoiseState(NoiseState):
    """Immutable noise state: step counter and key (reference ``_gaussian.py:65-79``)."""

    _step_counter: int
    _rng_key: RngKey


def _validate_stddev(std) -> None:
    if isinstance(std, PerGroup):
        for name, v in std.values.items():
            if v < 0:
                raise ConfigurationError(
                    "noise standard deviation must be non-negative for all groups, "
                    f"got {v} for group '{name}'"
                )
    elif std < 0:
        raise ConfigurationError(f"noise standard deviation must be non-negative, got {std}")


def paired_noise_stddevs(noise_multiplier: float, *, first, second):
    """Joint allocation of the paired release (reference noise_allocation.py:148-252):
    ``S = sum(first) + sum(second)``, ``sigma = nm * sqrt(delta * S)`` per stream."""
    if isinstance(first, PerGroup) != isinstance(second, PerGroup):
        raise InputTypeError(
            "paired_noise_stddevs requires both streams to have the same kind; got "
            f"first={type(first).__name__}, second={type(second).__name__}."
        )
    if noise_multiplier < 0:
        raise ConfigurationError(f"noise_multiplier must be non-negative, got {noise_multiplier}")

    def total(v):
        return float(sum(v.values.values())) if isinstance(v, PerGroup) else float(v)

    for label, v in (("first", first), ("second", second)):
        vals = v.values.values() if isinstance(v, PerGroup) else [v]
        for x in vals:
            if x < 0:
                raise ConfigurationError(f"{label} must be non-negative, got {x}.")
    s = total(first) + total(second)

    def scale(v):
        if isinstance(v, PerGroup):
            return PerGroup(v.groups, {k: noise_multiplier * math.sqrt(x * s) for k, x in v.values.items()})
        return noise_multiplier * math.sqrt(float(v) * s)

    return scale(first), scale(second)


def _leaf_std(std, path) -> float:
    return std.for_path(path) if isinstance(std, PerGroup) else float(std)


def add_noise_tree(tree: Any, std, step_key: RngKey, *, stream: str,
                   compute_dtype: torch.dtype = torch.float32) -> Any:
    """Add N(0, std^2) to every tensor leaf; leaf order is the flatten order."""
    _validate_stddev(std)
    paths, leaves, treedef = tree_flatten_with_paths(tree)
    gen = generator_from_key(step_key) if stream == "reference" else None
    out = []
    for index, (path, leaf) in enumerate(zip(paths, leaves)):
        if not isinstance(leaf, torch.Tensor):
            if isinstance(std, PerGroup):
                raise InputTypeError(
                    "gaussian_noise with PerGroup stddev expects tensor leaves; got "
                    f"{type(leaf).__name__} at path {path!r}."
                )
            out.append(leaf)
            continue
        s = _leaf_std(std, path)
        if s == 0:
            out.append(leaf)  # the reference returns the centre itself, no draw
            continue
        if leaf.dtype not in _SUPPORTED_COMPUTE:
            raise OperationError(
                f"leaf dtype {leaf.dtype} is not supported (float16, bfloat16, float32, float64)")
        if stream == "reference":
            draw = torch.randn(tuple(leaf.shape), dtype=compute_dtype, generator=gen)
            draw = draw.pin_memory().to(leaf.device, non_blocking=True)
            out.append(ops.add_noise(leaf, s, mode=nat.NOISE_INJECTED, noise=draw,
                                     compute_dtype=compute_dtype))
        else:
            out.append(ops.add_noise(leaf, s, mode=nat.NOISE_PHILOX, seed=step_key.seed,
                                     leaf_id=index, compute_dtype=compute_dtype))
    return tree_unflatten(treedef, out)


def gaussian_noise(
    *,
    noise_multiplier: float,
    key: RngKey,
    compute_dtype: torch.dtype = torch.float32,
    stream: str = "reference",
):
    """Create ``(noise_fn, state)``; see the module docstring."""
    if noise_multiplier is None:
        raise ConfigurationError("gaussian_noise() requires noise_multiplier.")
    nm = float(noise_multiplier)
    if nm < 0:
        raise ConfigurationError(f"noise_multiplier must be non-negative, got {noise_multiplier}")
    if not isinstance(compute_dtype, torch.dtype):
        raise InputTypeError(
            f"compute_dtype must be torch.dtype, got {type(compute_dtype).__name__}"
        )
    if compute_dtype not in _SUPPORTED_COMPUTE:
        raise ConfigurationError(
            "compute_dtype must be one of torch.float16, torch.bfloat16, torch.float32, or "
            f"torch.float64; got {compute_dtype}."
        )
    if not isinstance(key, RngKey):
        raise InputTypeError(f"key must be RngKey, got {type(key)}")
    if stream not in STREAMS:
        raise ConfigurationError(f"stream must be one of {STREAMS}, got {stream!r}")

    state = GaussianNoiseState(_step_counter=0, _rng_key=key)

    def clipped_stddev(c: ClippedPytree):
        if isinstance(c.max_norm, PerGroup):
            return per_group_noise_stddev(c.max_norm, nm)
        eff = 0.0 if nm == 0.0 else nm * c.max_norm
        _validate_stddev(eff)
        return eff

    def impl(grads, st):
        nxt = GaussianNoiseState(_step_counter=st._step_counter + 1, _rng_key=st._rng_key)
        if isinstance(grads, SecondMomentClippingOutput):
            first, second = grads.grads, grads.squared_grads
            if not isinstance(first, ClippedPytree):
                raise InputTypeError("SecondMomentClippingOutput.grads must be a ClippedPytree.")
            if not isinstance(second, ClippedPytree):
                raise InputTypeError(
                    "SecondMomentClippingOutput.squared_grads must be a ClippedPytree."
                )
            s1, s2 = paired_noise_stddevs(nm, first=first.max_norm, second=second.max_norm)
            k1 = fold_in(st._rng_key, GAUSSIAN_STREAM_FOLD, PAIRED_FIRST_STREAM_FOLD, st._step_counter)
            k2 = fold_in(st._rng_key, GAUSSIAN_STREAM_FOLD, PAIRED_SECOND_STREAM_FOLD, st._step_counter)
            n1 = add_noise_tree(first.pytree, s1, k1, stream=stream, compute_dtype=compute_dtype)
            n2 = add_noise_tree(second.pytree, s2, k2, stream=stream, compute_dtype=compute_dtype)
            return (
                SecondMomentNoiseOutput(
                    NoisedPytree(pytree=n1, max_norm=first.max_norm, noise_stddev=s1),
                    NoisedPytree(pytree=n2, max_norm=second.max_norm, noise_stddev=s2),
                ),
                nxt,
            )
        if isinstance(grads, NoisedPytree):
            raise InputTypeError(
                "gaussian_noise expects ClippedPytree inputs, not NoisedPytree values that "
                "have already passed through a noise mechanism."
            )
        if not isinstance(grads, ClippedPytree):
            raise InputTypeError(
                "gaussian_noise expects ClippedPytree inputs. Wrap manual values with "
                "opake_amd.types.clipped(...)."
            )
        std = clipped_stddev(grads)
        step_key = fold_in(st._rng_key, GAUSSIAN_STREAM_FOLD, st._step_counter)
        noisy = add_noise_tree(grads.pytree, std, step_key, stream=stream,
                               compute_dtype=compute_dtype)
        return NoisedPytree(pytree=noisy, max_norm=grads.max_norm, noise_stddev=std), nxt

    def noise_fn(grads, st):
        with record_function("opake::gaussian_noise"):
            return impl(grads, st)

    # Configuration, read by the fused clip+noise paths.
    noise_fn.noise_multiplier = nm
    noise_fn.stream = stream
    noise_fn.compute_dtype = compute_dtype
    noise_fn.clipped_stddev = clipped_stddev
    return noise_fn, state


def step_key_for(state: GaussianNoiseState) -> RngKey:
    """The key of the next single-stream draw for ``state``."""
    return fold_in(state._rng_key, GAUSSIAN_STREAM_FOLD, state._step_counter)


__all__ = [
    "GAUSSIAN_STREAM_FOLD",
    "GaussianNoiseState",
    "add_noise_tree",
    "gaussian_noise",
    "paired_noise_stddevs",
    "step_key_for",
]
