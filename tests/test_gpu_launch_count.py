"""The fused clip-and-sum's launch count does not grow with the number of
leaves (GPU test) -- the reference's contract for its fused kernel
(packages/opake-patches/tests/kernels/test_clip_sum.py:337-362): the same
``clipped_fun`` call over 6 and over 60 stacked leaves (float32, and mixed
float32 / bfloat16) issues the same number of device kernels, counted with
``torch.profiler`` after a warm-up call that builds and caches the tile plans
and pointer tables.
"""

from __future__ import annotations

import pytest
import torch

from opake_amd.clipping import clipped_fun

pytestmark = pytest.mark.gpu


def _tree(dev, B, n_leaves, *, mixed, seed):
    g = torch.Generator().manual_seed(seed)
    tree = {}
    for i in range(n_leaves):
        shape = (B, 1 + (i * 37) % 300, 1 + (i * 11) % 5)
        dtype = torch.bfloat16 if mixed and i % 2 else torch.float32
        tree[f"leaf{i:03d}"] = torch.randn(shape, generator=g).to(dtype).to(dev)
    return tree


def _kernels_per_call(fn, tree, state):
    fn(tree, state=state)  # warm-up: tile plans and device tables
    torch.cuda.synchronize()
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        fn(tree, state=state)
        torch.cuda.synchronize()
    cuda = torch.autograd.DeviceType.CUDA
    names = [e.name for e in prof.events() if e.device_type == cuda]
    return len(names), names


@pytest.mark.parametrize("mixed", [False, True], ids=["fp32", "mixed"])
def test_launches_do_not_grow_with_the_number_of_leaves(dev, mixed):
    counts = []
    for n_leaves in (6, 60):
        fn, state = clipped_fun(lambda v: v, batch_argnums=0, clipping_norm=1.0,
                                return_aux=True)
        count, names = _kernels_per_call(fn, _tree(dev, 4, n_leaves, mixed=mixed, seed=5),
                                         state)
        counts.append(count)
        assert any("tile_sq_kernel" in n for n in names), names
        assert any("apply_sum_kernel" in n for n in names), names
    assert counts[0] == counts[1], counts
