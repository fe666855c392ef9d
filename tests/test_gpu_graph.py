"""HIP-graph replay of the ghost clip -> sum step.

``GraphedGhostClip`` captures ``ghost_clip_captured`` once per operand
signature and replays it.  Every replay is checked bit for bit against the
eager call on the same operands, over several replays with new operand values
and with the program's own eager work and synchronisations between them (a
recorded memset or a stale recorded copy would show up as a wrong replay).
Covered: dense Gram layers with bias, flat (T = 1) layers, narrow layers
(direct per-example gradients), row-segmented (MoE) layers and materialised
per-example gradients.
"""

from __future__ import annotations

import pytest
import torch

from opake_amd.clipping import DirectCapture, GraphedGhostClip, LinearCapture, ghost_clip_captured
from opake_amd.types import PerGroup

pytestmark = pytest.mark.gpu


def _captures(gen, dev, scale):
    def r(*shape, s=1.0, dtype=torch.bfloat16):
        return (torch.randn(*shape, generator=gen) * s * scale).to(dtype).to(dev)

    B, T = 4, 128
    return [
        LinearCapture("dense", r(B, T, 64), r(B, T, 96, s=0.02), has_bias=True),
        LinearCapture("flat", r(B, 40, dtype=torch.float32), r(B, 24, s=0.1, dtype=torch.float32)),
        LinearCapture("adapter", r(B, T, 256), r(B, T, 8, s=0.05)),
        LinearCapture("expert", r(300, 64), r(300, 128, s=0.02), segments=[100, 0, 130, 70]),
        DirectCapture({"norm.weight": r(B, 64, s=0.3)}),
    ]


@pytest.mark.parametrize("per_group", [False, True])
def test_graph_replays_match_eager(dev, per_group):
    gen = torch.Generator().manual_seed(0)
    names = ["adapter.weight", "dense.bias", "dense.weight", "expert.weight", "flat.weight",
             "norm.weight"]
    C = (PerGroup({n: ("a" if n.startswith(("dense", "flat")) else "b") for n in names},
                  {"a": 0.5, "b": 0.2}) if per_group else 0.5)
    graphed = GraphedGhostClip(clipping_norm=C, normalize_by=4.0, dtype=torch.float32)
    for step in range(4):
        caps = _captures(gen, dev, 1.0 + step)
        got = graphed(caps)
        # Eager work between replays, then the eager reference on the same operands.
        torch.randn(1 << 20, device=dev).sum().item()
        want = ghost_clip_captured(caps, clipping_norm=C, normalize_by=4.0, dtype=torch.float32)
        torch.cuda.synchronize()
        assert sorted(got.pytree) == names
        for n in names:
            assert torch.equal(got.pytree[n], want.pytree[n]), (step, n)
        assert got.max_norm == want.max_norm
    assert graphed.captures == 1 and graphed.replays == 4
