"""GPU parity of every storage and compute dtype of the clip-and-sum and noise
paths, against the CPU oracle on the same inputs.

Leaves of float16, bfloat16, float32 and float64 (alone and mixed) go through
the materialised-leaf seam and ``clipped_fun`` with ``compute_dtype`` None or
each of the four floating dtypes (``_pytree.py:84-204``,
``_clipped_fun.py:91-148``); ``clip_pytree`` takes the same compute dtypes;
``gaussian_noise(compute_dtype=...)`` adds the reference stream bit for bit
(``_gaussian.py:188-204``: ``torch.randn(dtype=compute_dtype)`` on the CPU
generator, arithmetic in the compute dtype, cast back).

Tolerances: norms (reported in the reduction dtype) 1e-6 relative when the
reduction runs in float32, 1e-12 in float64, one rounding of a 16-bit
reduction dtype; batch sums within 8 units in the last place
of the coarsest dtype they pass through, relative to the largest entry (they
differ from torch's in summation order, which can move a rounding by a unit).
Injected reference-stream noise is compared bit for bit.
"""

from __future__ import annotations

import math

import pytest
import torch

from opake_amd import clipping as cl
from opake_amd.noise import gaussian_noise
from opake_amd.random import key
from opake_amd.types import clipped
from oracle import clip_oracle, noise_oracle

pytestmark = pytest.mark.gpu

F16, BF16, F32, F64 = torch.float16, torch.bfloat16, torch.float32, torch.float64


class _Scale:
    def __init__(self, kind, gamma=0.0):
        self.kind, self.gamma = kind, gamma


def _reduce_for(compute_dtype, output_dtype=None):
    """The reference's reduce_leaf (``_sum_clipped_tensor``, _clipped_fun.py:112-132)."""

    def reduce_leaf(x):
        acc = compute_dtype
        if acc is None and x.dtype in (F16, BF16):
            acc = F32
        out = torch.sum(x, dim=0, dtype=acc)
        return out.to(output_dtype or x.dtype)

    return reduce_leaf


def _coarsest(*dtypes):
    return max((d for d in dtypes if d is not None), key=lambda d: torch.finfo(d).eps)


def _close(got, want, *dtypes):
    """Within 8 units in the last place of the coarsest dtype the value went
    through (storage, reduction or output dtype), relative to the largest
    entry: the batch sums differ from torch's only in summation order."""
    got, want = got.cpu().double(), want.double()
    eps = torch.finfo(_coarsest(*dtypes)).eps
    scale = want.abs().max().item() if want.numel() else 0.0
    torch.testing.assert_close(got, want, rtol=8 * eps, atol=8 * eps * scale)


def _check_norms(got, want, acc):
    """Diagnostic norms come in the reduction dtype (``_streaming.py:174-180``):
    1e-6 relative of the fp64 norm for float32, 1e-12 for float64, and one
    rounding of a 16-bit reduction dtype."""
    assert got.dtype == acc
    if acc in (F16, BF16):
        torch.testing.assert_close(got.cpu().double(), want.to(acc).double(),
                                   rtol=torch.finfo(acc).eps, atol=0)
    else:
        torch.testing.assert_close(got.cpu().double(), want, rtol=1e-6 if acc == F32 else 1e-12,
                                   atol=0)


def _tree(gen, B, dtypes):
    shapes = [(5, 7), (2500,), (11,), (3, 2048), (1,)]
    tree = {}
    for i, shape in enumerate(shapes):
        dt = dtypes[i % len(dtypes)]
        scale = torch.exp(torch.randn(B, *([1] * len(shape)), generator=gen))
        tree[f"p{i}"] = (torch.randn(B, *shape, generator=gen) * scale * 0.05).to(dt)
    return tree


DTYPE_SETS = [[F16], [F64], [F16, F32, F64, BF16]]


@pytest.mark.parametrize("dtypes", DTYPE_SETS, ids=["f16", "f64", "mixed"])
@pytest.mark.parametrize("compute_dtype", [None, F16, BF16, F32, F64],
                         ids=["none", "c16", "cbf16", "c32", "c64"])
@pytest.mark.parametrize("second_moment", [False, True])
def test_leaf_backend_every_dtype(dev, dtypes, compute_dtype, second_moment):
    gen = torch.Generator().manual_seed(len(dtypes) + 17 * second_moment)
    B = 7
    tree = _tree(gen, B, dtypes)
    tree["p1"][2, 17] = math.nan
    tree["p3"][4, 0, 3] = -math.inf
    names = sorted(tree)
    C = clip_oracle.conservative_bound(0.5)
    res = clip_oracle.stream_clip_and_sum([tree[n] for n in names], C, return_aux=True,
                                          compute_dtype=compute_dtype,
                                          second_moment=second_moment)
    reduce_leaf = _reduce_for(compute_dtype)
    # The oracle's batch sum with the same reduce_leaf semantics.
    dev_tree = {k: v.to(dev) for k, v in tree.items()}
    reduced, markers, sq, sqm, diag = cl.fused_stream_clip_and_sum(
        dev_tree, torch.tensor(C, device=dev), scale=_Scale("fixed"), batch_size=B,
        reduce_leaf=reduce_leaf, compute_dtype=compute_dtype, second_moment=second_moment,
        return_aux=True, return_stats=False)
    acc = res.acc_dtype
    for i, n in enumerate(names):
        assert reduced[n].dtype == tree[n].dtype, n
        assert markers[n].dtype == tree[n].dtype and markers[n].dim() == 0
        _close(reduced[n], res.reduced[i], tree[n].dtype, compute_dtype)
        if second_moment:
            assert sq[n].dtype == tree[n].dtype and sqm[n].dtype == tree[n].dtype
            _close(sq[n], res.squared[i], tree[n].dtype, compute_dtype)
    _check_norms(diag["norms"], res.norms, acc)
    # ||stored||: the reference squares and sums in the reduction dtype (its
    # roundings for a 16-bit one), the kernels in fp64 and round once.
    rtol = 4 * torch.finfo(acc).eps if acc in (F16, BF16) else 1e-5
    torch.testing.assert_close(diag["clipped_norms"].cpu().double(),
                               res.clipped_norms.double(), rtol=rtol, atol=1e-7)


@pytest.mark.parametrize("leaf_dtype,output_dtype", [(F16, F32), (BF16, F64), (F64, F32),
                                                     (F32, F64), (F32, F16)])
def test_leaf_backend_output_dtypes(dev, leaf_dtype, output_dtype):
    gen = torch.Generator().manual_seed(3)
    B = 6
    tree = _tree(gen, B, [leaf_dtype])
    names = sorted(tree)
    C = clip_oracle.conservative_bound(0.3)
    res = clip_oracle.stream_clip_and_sum([tree[n] for n in names], C,
                                          reduce_dtype={leaf_dtype: output_dtype})
    reduced, _, _, _, _ = cl.fused_stream_clip_and_sum(
        {k: v.to(dev) for k, v in tree.items()}, torch.tensor(C, device=dev),
        scale=_Scale("auto_s", 0.01) if leaf_dtype == F64 else _Scale("fixed"), batch_size=B,
        reduce_leaf=_reduce_for(None, output_dtype), compute_dtype=None, second_moment=False,
        return_aux=False, return_stats=False)
    if leaf_dtype == F64:  # AUTO-S for this case: the oracle again, with AUTO-S
        res = clip_oracle.stream_clip_and_sum([tree[n] for n in names], C, kind="auto_s",
                                              gamma=0.01, reduce_dtype={leaf_dtype: output_dtype})
    for i, n in enumerate(names):
        assert reduced[n].dtype == output_dtype
        _close(reduced[n], res.reduced[i], leaf_dtype, output_dtype)


@pytest.mark.parametrize("dtype", [F16, F64])
@pytest.mark.parametrize("compute_dtype", [None, F32, F64])
@pytest.mark.parametrize("microbatch", [None, 3])
def test_clipped_fun_fp16_fp64(dev, dtype, compute_dtype, microbatch):
    gen = torch.Generator().manual_seed(5)
    B = 8
    x = (torch.randn(B, 40, generator=gen) * torch.exp(torch.randn(B, 1, generator=gen))).to(dtype)

    def f(v):
        return {"a": v * 2, "b": v[:3]}

    fn, st = cl.clipped_fun(f, clipping_norm=1.0, compute_dtype=compute_dtype,
                            microbatch_size=microbatch, return_aux=True)
    (out, aux), _ = fn(x.to(dev), state=st)
    per = [x * 2, x[:, :3]]  # sorted leaf order: "a", "b"
    C = clip_oracle.conservative_bound(1.0)
    res = clip_oracle.stream_clip_and_sum(per, C, compute_dtype=compute_dtype, return_aux=True)
    assert out.pytree["a"].dtype == dtype and out.pytree["b"].dtype == dtype
    if microbatch is None:
        _close(out.pytree["a"], res.reduced[0], dtype, compute_dtype)
        _close(out.pytree["b"], res.reduced[1], dtype, compute_dtype)
    else:
        # Chunk sums in the accumulation dtype, added, cast once: within the
        # output dtype's rounding of the full-batch sum.
        torch.testing.assert_close(out.pytree["a"].cpu().double(), res.reduced[0].double(),
                                   rtol=8 * torch.finfo(dtype).eps, atol=1e-3)
    acc = res.acc_dtype
    _check_norms(aux.norms, res.norms, acc)
    assert aux.clipping_rate * B == clip_oracle.num_clipped(res.norms.to(acc), 1.0)


@pytest.mark.parametrize("dtype", [F16, BF16, F32, F64])
@pytest.mark.parametrize("compute_dtype", [None, F16, F32, F64])
def test_clip_pytree_compute_dtypes(dev, dtype, compute_dtype):
    gen = torch.Generator().manual_seed(9)
    leaves = [(torch.randn(3, 5, generator=gen) * 2).to(dtype),
              (torch.randn(700, generator=gen)).to(dtype)]
    tree = {"a": leaves[0].to(dev), "b": leaves[1].to(dev)}
    out, aux = cl.clip_pytree(tree, 1.5, compute_dtype=compute_dtype)
    want, norm = clip_oracle.clip_pytree_scalar(leaves, 1.5, compute_dtype=compute_dtype)
    assert out["a"].dtype == dtype and out["b"].dtype == dtype
    # One example: the stored values themselves, the same roundings (the
    # scale can differ by the fp64 order of the norm's sum: a unit or so).
    acc = clip_oracle.resolve_compute_dtype_for_reduction([dtype], compute_dtype)
    _close(out["a"], want[0], dtype)
    _close(out["b"], want[1], dtype)
    assert float(torch.linalg.vector_norm(out["b"].double()) ** 2
                 + torch.linalg.vector_norm(out["a"].double()) ** 2) <= 1.5 ** 2
    torch.testing.assert_close(aux.norm.cpu().double(), norm.double(),
                               rtol=1e-6 if acc != F64 else 1e-12, atol=0)


@pytest.mark.parametrize("leaf_dtype", [F16, BF16, F32, F64])
@pytest.mark.parametrize("compute_dtype", [F16, BF16, F32, F64])
def test_gaussian_noise_reference_stream_every_compute_dtype(dev, leaf_dtype, compute_dtype):
    gen = torch.Generator().manual_seed(21)
    tree = {"w": (torch.randn(37, 19, generator=gen) * 0.1).to(leaf_dtype),
            "b": (torch.randn(19, generator=gen) * 0.1).to(leaf_dtype)}
    noise_fn, st = gaussian_noise(noise_multiplier=0.7, key=key(3), compute_dtype=compute_dtype)
    out, st2 = noise_fn(clipped({k: v.to(dev) for k, v in tree.items()}, max_norm=1.3), st)
    assert st2._step_counter == 1
    seed = noise_oracle.step_seed(key(3).seed, 0)
    leaves = [tree["b"], tree["w"]]  # sorted keys
    draws = noise_oracle.draws_for(leaves, seed, compute_dtype=compute_dtype)
    for name, leaf, z in zip(["b", "w"], leaves, draws):
        want = noise_oracle.sample(leaf, 0.7 * 1.3, z, compute_dtype=compute_dtype)
        got = out.pytree[name]
        assert got.dtype == leaf_dtype
        assert torch.equal(got.cpu(), want), (name, (got.cpu().double() - want.double()).abs().max())


@pytest.mark.parametrize("leaf_dtype", [F16, F64])
@pytest.mark.parametrize("compute_dtype", [F16, BF16, F64])
def test_gaussian_noise_device_stream_every_compute_dtype(dev, leaf_dtype, compute_dtype):
    # The device stream in another compute dtype: the float32 Philox normal of
    # each element rounded to the compute dtype, then the same arithmetic.
    x = torch.zeros(512, 64, dtype=leaf_dtype, device=dev)
    noise_fn, st = gaussian_noise(noise_multiplier=1.0, key=key(4), compute_dtype=compute_dtype,
                                  stream="device")
    out, _ = noise_fn(clipped({"w": x}, max_norm=1.0), st)
    noise32, _ = gaussian_noise(noise_multiplier=1.0, key=key(4), stream="device")[0](
        clipped({"w": torch.zeros(512, 64, dtype=F32, device=dev)}, max_norm=1.0), st)
    z = noise32.pytree["w"].double()
    want = z.to(compute_dtype).to(leaf_dtype)  # 0 + 1.0 * to_cd(z), cast back
    assert torch.equal(out.pytree["w"], want)
    v = out.pytree["w"].double()
    assert abs(v.mean().item()) < 0.02 and abs(v.std().item() - 1.0) < 0.02
