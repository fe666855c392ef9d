"""Golden vectors of the key derivation -- CPU only.

``tests/golden/rng_vectors.json`` holds outputs of the reference's own
``key`` / ``fold_in`` / ``split`` / ``generator_from_key``
(packages/opake-engine/src/opake/api/engine/random/_engine.py), recorded by
``tests/golden/gen_rng_vectors.py`` in the build container: negative and
>= 2^63 integers, integers at the edge of the 16-byte encoding, empty and
non-ASCII strings, the noise stream tags and chained folds, and the seed and
first draws of the torch generator of a step key.  Both the product
(``opake_amd.random``) and the oracle (``oracle/noise_oracle.py``) must
reproduce them exactly; a byte-order or separator mistake planted in the
oracle's hash must not.
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import pytest
import torch

from opake_amd import random as rng
from oracle import noise_oracle

FIXTURE = json.loads((Path(__file__).parent / "golden" / "rng_vectors.json").read_text())


def _datum(d):
    return int(d["int"]) if isinstance(d, dict) else d


def test_key():
    for case in FIXTURE["key"]:
        s = int(case["seed_in"])
        assert rng.key(s).seed == int(case["seed"])
        assert noise_oracle.key_seed(s) == int(case["seed"])


def test_fold_in():
    assert len(FIXTURE["fold_in"]) >= 50
    for case in FIXTURE["fold_in"]:
        k = rng.key(int(case["seed_in"]))
        d = _datum(case["data"])
        assert rng.fold_in(k, d).seed == int(case["seed"]), case
        assert noise_oracle.fold_in_seed(k.seed, d) == int(case["seed"]), case


def test_chained_fold_in():
    for case in FIXTURE["chains"]:
        k = rng.key(int(case["seed_in"]))
        data = [_datum(d) for d in case["data"]]
        assert rng.fold_in(k, *data).seed == int(case["seed"])
        assert noise_oracle.fold_in_seed(k.seed, *data) == int(case["seed"])
    # The step seeds of the noise streams (single and paired).
    by = {(c["seed_in"], tuple(str(_datum(d)) for d in c["data"])): int(c["seed"])
          for c in FIXTURE["chains"]}
    assert noise_oracle.step_seed(0, 1) == by[("0", ("opake.dpsgd.gaussian", "1"))]
    assert noise_oracle.step_seed(42, 0, "opake.paired.first") == \
        by[("42", ("opake.dpsgd.gaussian", "opake.paired.first", "0"))]


def test_split():
    for case in FIXTURE["split"]:
        kids = rng.split(rng.key(int(case["seed_in"])), case["num"])
        assert [k.seed for k in kids] == [int(s) for s in case["seeds"]]


def test_generator_from_key_seed_and_draws():
    for case in FIXTURE["generator"]:
        k = rng.fold_in(rng.key(int(case["seed_in"])), "opake.dpsgd.gaussian", case["step"])
        assert k.seed == int(case["key_seed"])
        gen = rng.generator_from_key(k)
        assert gen.initial_seed() == int(case["torch_seed"])
        draws = torch.randn(8, dtype=torch.float32, generator=gen)
        assert draws.tolist() == case["randn8"]
        seed = noise_oracle.step_seed(int(case["seed_in"]), case["step"])
        (odraw,) = noise_oracle.draws_for([torch.zeros(8)], seed)
        assert odraw.tolist() == case["randn8"]


@pytest.mark.parametrize("mistake", ["big_endian", "no_separator", "no_tag"])
def test_planted_hash_mistakes_fail(mistake):
    def digest(seed, datum):
        h = hashlib.blake2b(digest_size=8)
        for part in (seed, datum):
            if isinstance(part, int):
                if mistake != "no_tag":
                    h.update(b"i")
                h.update(part.to_bytes(16, "big" if mistake == "big_endian" else "little",
                                       signed=True))
            else:
                if mistake != "no_tag":
                    h.update(b"s")
                h.update(str(part).encode("utf-8"))
            if mistake != "no_separator":
                h.update(b"|")
        return int.from_bytes(h.digest(), "little")

    # (with a zero seed the byte order shows only in a nonzero integer datum,
    # so only the cases of nonzero seeds must all differ)
    cases = [c for c in FIXTURE["fold_in"] if mistake != "big_endian" or c["seed_in"] != "0"]
    assert len(cases) >= 36
    for c in cases:
        assert digest(int(c["seed_in"]) & ((1 << 64) - 1), _datum(c["data"])) != int(c["seed"])
