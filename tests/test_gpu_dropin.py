"""Drop-in keywords of the clipping factories on the GPU.

* ``compute_dtype`` (packages/opake-engine/src/opake/api/engine/clipping/
  _clipped_grad.py:100, _pytree.py:84-108, _clipped_fun.py:91-170): float32
  gives the default's bits for bfloat16 and float32 leaves; bfloat16 (with
  bfloat16 leaves) squares, guards and multiplies in bfloat16, float64
  squares and multiplies in float64 -- against the streaming oracle run with
  the same compute dtype (every other combination: tests/test_gpu_dtypes.py).
* ``pre_clipping_transform`` (_clipped_grad.py:97,285, _auto.py:222): applied
  to each example's gradient before clipping, against the oracle clipping the
  transformed per-example gradients, including a transform that changes the
  pytree's structure.
"""

from __future__ import annotations

import pytest
import torch

from opake_amd.clipping import auto_clipped_grad, clipped_fun, clipped_grad
from oracle import clip_oracle

pytestmark = pytest.mark.gpu


def _rel(got, want):
    got, want = got.double().cpu(), want.double().cpu()
    return ((got - want).norm() / want.norm().clamp_min(1e-300)).item()


def _tree(dev, dtype, B=6, seed=0):
    g = torch.Generator().manual_seed(seed)
    return {"a": (torch.randn(B, 300, 7, generator=g) * 0.1).to(dtype).to(dev),
            "b": (torch.randn(B, 5000, generator=g) * 0.01).to(dtype).to(dev)}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_compute_dtype_float32_is_the_default(dev, dtype):
    tree = _tree(dev, dtype)
    outs = []
    for cd in (None, torch.float32):
        fn, st = clipped_fun(lambda v: v, batch_argnums=0, clipping_norm=0.3,
                             compute_dtype=cd, return_aux=True)
        (res, aux), _ = fn(tree, state=st)
        outs.append((res.pytree, aux.norms))
    for k in tree:
        assert torch.equal(outs[0][0][k], outs[1][0][k])
    assert torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("microbatch", [None, 4])
def test_compute_dtype_bfloat16_matches_oracle(dev, microbatch):
    tree = _tree(dev, torch.bfloat16, B=8, seed=3)
    fn, st = clipped_fun(lambda v: v, batch_argnums=0, clipping_norm=0.3,
                         compute_dtype=torch.bfloat16, return_aux=True,
                         microbatch_size=microbatch)
    (res, aux), _ = fn(tree, state=st)
    names = sorted(tree)
    leaves = [tree[n].cpu() for n in names]
    want = clip_oracle.stream_clip_and_sum(leaves, clip_oracle.conservative_bound(0.3),
                                           compute_dtype=torch.bfloat16)
    for n, w in zip(names, want.reduced):
        assert res.pytree[n].dtype == torch.bfloat16
        assert _rel(res.pytree[n], w) < 2e-2, n
    # The diagnostic norms come in the reduction dtype (_streaming.py:174-180).
    assert aux.norms.dtype == torch.bfloat16
    torch.testing.assert_close(aux.norms.cpu().double(), want.norms.to(torch.bfloat16).double(),
                               rtol=2 ** -8, atol=0)
    # The bf16 guard and multiply: every stored example's norm is within C.
    fn2, st2 = clipped_fun(lambda v: v, batch_argnums=0, clipping_norm=0.3,
                           compute_dtype=torch.bfloat16, return_aux=True)
    (_, aux2), _ = fn2(tree, state=st2)
    assert torch.all(aux2.clipped_norms.double() <= 0.3 * (1 + 1e-6))


def test_compute_dtype_float64_matches_oracle(dev):
    tree = _tree(dev, torch.float32, B=8, seed=4)
    fn, st = clipped_fun(lambda v: v, batch_argnums=0, clipping_norm=0.3,
                         compute_dtype=torch.float64, return_aux=True)
    (res, aux), _ = fn(tree, state=st)
    names = sorted(tree)
    want = clip_oracle.stream_clip_and_sum([tree[n].cpu() for n in names],
                                           clip_oracle.conservative_bound(0.3),
                                           compute_dtype=torch.float64)
    for n, w in zip(names, want.reduced):
        assert res.pytree[n].dtype == torch.float32
        torch.testing.assert_close(res.pytree[n].cpu(), w, rtol=1e-6, atol=1e-9)
    assert aux.norms.dtype == torch.float64
    torch.testing.assert_close(aux.norms.cpu(), want.norms, rtol=1e-12, atol=0)


def _loss(p, x):
    return 0.5 * ((x @ p["w"].T + p["b"]) ** 2).sum()


def _params(dev):
    g = torch.Generator().manual_seed(1)
    return {"w": torch.randn(3, 4, generator=g).to(dev), "b": torch.randn(3, generator=g).to(dev)}


def _per_example(p, xs):
    from torch.func import grad, vmap
    return vmap(grad(_loss), in_dims=(None, 0))(p, xs)


@pytest.mark.parametrize("factory", ["clipped_grad", "auto_clipped_grad"])
def test_pre_clipping_transform_matches_oracle(dev, factory):
    p = _params(dev)
    xs = torch.randn(10, 2, 4, generator=torch.Generator().manual_seed(2)).to(dev)

    def transform(g):  # a diagonal preconditioner on w, b dropped
        return {"w": g["w"] * torch.tensor([1.0, 2.0, 0.5, 3.0], device=g["w"].device)}

    if factory == "clipped_grad":
        fn, st = clipped_grad(_loss, clipping_norm=0.7, pre_clipping_transform=transform)
    else:
        fn, st = auto_clipped_grad(_loss, R=0.7, gamma=0.05, pre_clipping_transform=transform)
    res, _ = fn(p, xs, state=st)
    assert set(res.pytree) == {"w"}
    per = transform(_per_example(p, xs))
    want = clip_oracle.stream_clip_and_sum(
        [per["w"].cpu()], clip_oracle.conservative_bound(0.7),
        kind="fixed" if factory == "clipped_grad" else "auto_s", gamma=0.05)
    torch.testing.assert_close(res.pytree["w"].cpu(), want.reduced[0], rtol=1e-5, atol=1e-6)
