"""CPU restatement of the reference's key derivation and Gaussian noise.

TEST INFRASTRUCTURE: imported only by tests/, smoke() and bench.py's CPU
baseline.

* ``key`` / ``fold_in`` / ``split``: packages/opake-engine/src/opake/api/
  engine/random/_engine.py:22-137 (BLAKE2b-64 over tagged parts).
* ``reference_noise``: the draw of packages/opake-dpsgd/src/opake/api/dpsgd/
  noise/_gaussian.py:188-229,299-343 -- step key
  ``fold_in(key, "opake.dpsgd.gaussian", step)``, one CPU ``torch.Generator``
  seeded with ``seed % (2^63 - 1)``, ``torch.randn(shape, float32)`` per leaf in
  flatten order (dict keys sorted), ``center.float() + std * noise`` cast back.
* ``per_group_noise_stddev``: engine/noise_allocation.py:44-110.
"""

from __future__ import annotations

import hashlib
import math

import torch

GAUSSIAN_STREAM_FOLD = "opake.dpsgd.gaussian"
_U64 = (1 << 64) - 1


def _digest(seed: int, datum) -> int:
    h = hashlib.blake2b(digest_size=8)
    for part in (seed, datum):
        if isinstance(part, int):
            h.update(b"i")
            h.update(part.to_bytes(16, "little", signed=True))
        else:
            h.update(b"s")
            h.update(str(part).encode("utf-8"))
        h.update(b"|")
    return int.from_bytes(h.digest(), "little")


def key_seed(seed: int) -> int:
    return seed & _U64


def fold_in_seed(seed: int, *data) -> int:
    for d in data:
        seed = _digest(seed, d)
    return seed


def step_seed(base_seed: int, step: int, *streams: str) -> int:
    """Seed of the step key: fold_in(key, GAUSSIAN_STREAM_FOLD, *streams, step)."""
    return fold_in_seed(base_seed, GAUSSIAN_STREAM_FOLD, *streams, step)


def generator_for(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed % (2**63 - 1))


def flatten_sorted(tree):
    """Leaves in optree order for dict/list/tuple trees (dict keys sorted)."""
    if isinstance(tree, dict):
        out = []
        for k in sorted(tree):
            out.extend(flatten_sorted(tree[k]))
        return out
    if isinstance(tree, (list, tuple)):
        out = []
        for v in tree:
            out.extend(flatten_sorted(v))
        return out
    if tree is None:
        return []
    return [tree]


def draws_for(leaves, seed: int, compute_dtype=torch.float32):
    """The raw standard-normal tensors the reference draws, in order."""
    gen = generator_for(seed)
    return [torch.randn(tuple(l.shape), dtype=compute_dtype, generator=gen) for l in leaves]


def sample(center: torch.Tensor, std: float, noise: torch.Tensor,
           compute_dtype=torch.float32) -> torch.Tensor:
    """``_sample`` (_gaussian.py:188-204) given the drawn noise."""
    if std == 0:
        return center
    in_dtype = center.dtype
    c = center.to(compute_dtype) if in_dtype != compute_dtype else center
    out = c + std * noise.to(c.device)
    return out.to(in_dtype) if in_dtype != compute_dtype else out


def per_group_noise_stddev(values: dict, nm: float) -> dict:
    if nm == 0.0:
        return dict.fromkeys(values, 0.0)
    total = sum(values.values())
    return {k: nm * math.sqrt(c * total) for k, c in values.items()}


__all__ = [
    "GAUSSIAN_STREAM_FOLD",
    "draws_for",
    "flatten_sorted",
    "fold_in_seed",
    "generator_for",
    "key_seed",
    "per_group_noise_stddev",
    "sample",
    "step_seed",
]
