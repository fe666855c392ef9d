"""Writes tests/golden/rng_vectors.json from the reference's key derivation.

Runs in the build container only (``/root/reference`` is not on the GPU box;
nothing imports this script).  It loads the reference module
``packages/opake-engine/src/opake/api/engine/random/_engine.py`` on its own --
its only dependencies are the standard library, torch and opake-base's
exception classes -- and records, for a fixed list of inputs, the outputs of
``key``, ``fold_in``, ``split`` and the seed and first draws of
``generator_from_key``: the functions behind the reference-stream noise
(``fold_in(key, "opake.dpsgd.gaussian", step)``, the paired tags
``"opake.paired.first"`` / ``"opake.paired.second"``) whose only other pins
are properties.  The fixture is data: inputs and expected outputs.

    python tests/golden/gen_rng_vectors.py
"""

from __future__ import annotations

import importlib.util
import json
import sys
from pathlib import Path

REF = Path("/root/reference/packages")
OUT = Path(__file__).resolve().parent / "rng_vectors.json"


def load_engine():
    sys.path.insert(0, str(REF / "opake-base" / "src"))
    path = REF / "opake-engine" / "src" / "opake" / "api" / "engine" / "random" / "_engine.py"
    spec = importlib.util.spec_from_file_location("_ref_rng_engine", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod
    spec.loader.exec_module(mod)
    return mod


SEEDS = [0, 1, 42, 7, -1, -12345, 2**32, 2**63 - 1, 2**63, 2**64 - 1, 2**64 + 5, -(2**63),
         123456789012345678901234567890]
DATA = [0, 1, 2, 17, -1, -(2**40), 2**63, 2**64 + 3, 2**126, -(2**127), "", "1", "0",
        "opake.dpsgd.gaussian", "opake.paired.first", "opake.paired.second",
        "mylab.rare_events", "ünïcødé ✓ 雪"]
CHAINS = [
    ["opake.dpsgd.gaussian", 0],
    ["opake.dpsgd.gaussian", 1],
    ["opake.dpsgd.gaussian", 99],
    ["opake.dpsgd.gaussian", "opake.paired.first", 0],
    ["opake.dpsgd.gaussian", "opake.paired.second", 0],
    ["opake.dpsgd.gaussian", "opake.paired.first", 5],
    [3, "opake.dpsgd.gaussian", 2],
    [1, 2, 3, 4],
]


def main():
    import torch

    eng = load_engine()
    out = {"source": "packages/opake-engine/src/opake/api/engine/random/_engine.py",
           "key": [], "fold_in": [], "chains": [], "split": [], "generator": []}
    for s in SEEDS:
        out["key"].append({"seed_in": str(s), "seed": str(eng.key(s).seed)})
    for s in (0, 42, 2**64 - 1):
        k = eng.key(s)
        for d in DATA:
            out["fold_in"].append({"seed_in": str(s), "data": d if isinstance(d, str) else
                                   {"int": str(d)}, "seed": str(eng.fold_in(k, d).seed)})
    for s in (0, 42):
        k = eng.key(s)
        for chain in CHAINS:
            out["chains"].append({"seed_in": str(s),
                                  "data": [d if isinstance(d, str) else {"int": str(d)}
                                           for d in chain],
                                  "seed": str(eng.fold_in(k, *chain).seed)})
    for s in (0, 9):
        for n in (1, 2, 5):
            out["split"].append({"seed_in": str(s), "num": n,
                                 "seeds": [str(c.seed) for c in eng.split(eng.key(s), n)]})
    for s in (0, 42):
        for step in (0, 1, 7):
            k = eng.fold_in(eng.key(s), "opake.dpsgd.gaussian", step)
            gen = eng.generator_from_key(k)
            draws = torch.randn(8, dtype=torch.float32, generator=gen)
            out["generator"].append({"seed_in": str(s), "step": step, "key_seed": str(k.seed),
                                     "torch_seed": str(gen.initial_seed()),
                                     "randn8": [float(x) for x in draws]})
    OUT.write_text(json.dumps(out, indent=1, ensure_ascii=False) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
