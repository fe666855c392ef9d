"""Explicit RNG keys with JAX-style semantics.

Same key derivation as the reference
(``packages/opake-engine/src/opake/api/engine/random/_engine.py:22-137``):
a key is a 64-bit seed; ``fold_in`` hashes ``(seed, datum)`` with
BLAKE2b-64, integers and strings taking disjoint encodings; ``split`` folds in
``0..n-1``; ``generator_from_key`` seeds a CPU ``torch.Generator`` with
``seed mod (2^63 - 1)``.  The derived 64-bit seed also keys the on-device
Philox stream of :func:`opake_amd.noise.gaussian_noise`.
"""

from __future__ import annotations

import dataclasses
import hashlib

import torch

from opake_amd.exceptions import ConfigurationError, InputTypeError

_MAX_TORCH_SEED = 2**63 - 1
_U64 = (1 << 64) - 1


def _hash64(*parts: object) -> int:
    """BLAKE2b (8-byte digest) over tagged parts: ``b"i"`` + 16-byte signed
    little-endian for ints, ``b"s"`` + UTF-8 for strings, each followed by
    ``b"|"``; the digest is read as a little-endian unsigned integer."""
    h = hashlib.blake2b(digest_size=8)
    for part in parts:
        if isinstance(part, int):
            h.update(b"i" + part.to_bytes(16, "little", signed=True))
        else:
            h.update(b"s" + str(part).encode("utf-8"))
        h.update(b"|")
    return int.from_bytes(h.digest(), "little", signed=False)


@dataclasses.dataclass(frozen=True)
class RngKey:
    seed: int
    impl: str = "opake_threefry_like"


def key(seed: int) -> RngKey:
    if not isinstance(seed, int) or isinstance(seed, bool):
        raise InputTypeError(f"seed must be int, got {type(seed)}")
    return RngKey(seed=seed & _U64)


def fold_in(rng_key: RngKey, *data: int | str) -> RngKey:
    if not isinstance(rng_key, RngKey):
        raise InputTypeError(f"rng_key must be RngKey, got {type(rng_key)}")
    if not data:
        raise ConfigurationError("fold_in requires at least one data argument")
    out = rng_key
    for d in data:
        if isinstance(d, bool) or not isinstance(d, (int, str)):
            raise InputTypeError(f"data must be int or str, got {type(d)}")
        out = RngKey(seed=_hash64(out.seed, d), impl=out.impl)
    return out


def split(rng_key: RngKey, num: int = 2) -> tuple[RngKey, ...]:
    if isinstance(num, bool) or not isinstance(num, int):
        raise InputTypeError(f"num must be int, got {type(num)}")
    if num < 1:
        raise ConfigurationError(f"num must be >= 1, got {num}")
    return tuple(fold_in(rng_key, i) for i in range(num))


def generator_from_key(rng_key: RngKey) -> torch.Generator:
    return torch.Generator().manual_seed(rng_key.seed % _MAX_TORCH_SEED)


__all__ = ["RngKey", "fold_in", "generator_from_key", "key", "split"]
