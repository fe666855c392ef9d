"""GPU parity of model-level ghost clipping on a Llama-style block.

``ghost_clipped_grad`` on a ``BlockLM`` (frozen embedding and head; the block's
fused qkv / o / gate_up / down projections by the Gram path, its two RMSNorm
weights by materialised per-example gradients) against the oracle: per-example
gradients of every block parameter from a loop of single-example backward
passes (float64), clipped and summed by the streaming oracle.  Tolerances:
1e-5 relative for float32, 2e-2 relative for bfloat16.
"""

from __future__ import annotations

import pytest
import torch

from opake_amd.clipping import auto_ghost_clipped_grad, ghost_clipped_grad
from opake_amd.noise import gaussian_noise
from opake_amd.random import key
from opake_amd.transformer import BlockLM, per_example_lm_loss
from opake_amd.types import NoisedPytree, PerGroup
from oracle import clip_oracle, ghost_oracle

pytestmark = pytest.mark.gpu


def _rel(got, want):
    got, want = got.double().cpu(), want.double().cpu()
    return ((got - want).norm() / want.norm().clamp_min(1e-300)).item()


def _case(dtype, vocab, d, heads, ffn, B, T, seed):
    torch.manual_seed(seed)
    ref = BlockLM(vocab, d, heads, ffn, dtype=torch.float64)
    with torch.no_grad():
        for p in ref.parameters():
            p.normal_(0.0, 0.05)
            if dtype == torch.bfloat16:
                p.copy_(p.to(torch.bfloat16).double())
    g = torch.Generator().manual_seed(seed + 1)
    ids = torch.randint(0, vocab, (B, T), generator=g)
    tgt = torch.randint(0, vocab, (B, T), generator=g)
    return ref, ids, tgt


def _groups(names):
    return PerGroup({n: ("attn" if any(k in n for k in ("qkv", ".o.", "attn_norm")) else "mlp")
                     for n in names}, {"attn": 0.3, "mlp": 0.2})


def _oracle(ref, ids, tgt, C, names, kind="fixed", gamma=0.0):
    per = ghost_oracle.per_example_grads_loop(ref, per_example_lm_loss, (ids,), tgt)
    leaves = [per[n].float() for n in names]
    if isinstance(C, PerGroup):
        groups = [C.groups[(n,)] for n in names]
        values = {k: clip_oracle.conservative_bound(v) for k, v in C.values.items()}
        return clip_oracle.stream_clip_and_sum(leaves, None, groups=groups, group_values=values,
                                               kind=kind, gamma=gamma, return_aux=True)
    return clip_oracle.stream_clip_and_sum(leaves, clip_oracle.conservative_bound(C), kind=kind,
                                           gamma=gamma, return_aux=True)


@pytest.mark.parametrize("per_group", [False, True])
def test_ghost_block_float32_matches_per_example_oracle(dev, per_group):
    ref, ids, tgt = _case(torch.float32, 61, 32, 4, 48, 3, 20, seed=0)
    model = BlockLM(61, 32, 4, 48, dtype=torch.float32).to(dev)
    model.load_state_dict({k: v.float() for k, v in ref.state_dict().items()})
    names = sorted(n for n, p in model.named_parameters() if p.requires_grad)
    assert len(names) == 6
    C = _groups(names) if per_group else 0.25
    res = _oracle(ref, ids, tgt, C, names)
    fn, st = ghost_clipped_grad(model, per_example_lm_loss, clipping_norm=C, normalize_by=3.0,
                                return_aux=True)
    (out, aux), _ = fn(ids.to(dev), tgt.to(dev), state=st)
    assert sorted(out.pytree) == names
    for i, n in enumerate(names):
        assert out.pytree[n].dtype == torch.float32
        assert _rel(out.pytree[n], res.reduced[i] / 3.0) < 1e-5, n
    if per_group:
        for gname in ("attn", "mlp"):
            torch.testing.assert_close(aux.group_norms[gname].cpu().double(),
                                       res.group_norms[gname], rtol=1e-5, atol=0)
    else:
        torch.testing.assert_close(aux.grad_norms.cpu().double(), res.norms, rtol=1e-5, atol=0)


def test_ghost_block_bf16_matches_per_example_oracle(dev):
    ref, ids, tgt = _case(torch.bfloat16, 100, 128, 4, 192, 4, 128, seed=3)
    model = BlockLM(100, 128, 4, 192, dtype=torch.bfloat16).to(dev)
    model.load_state_dict({k: v.to(torch.bfloat16) for k, v in ref.state_dict().items()})
    names = sorted(n for n, p in model.named_parameters() if p.requires_grad)
    res = _oracle(ref, ids, tgt, 0.05, names)
    fn, st = ghost_clipped_grad(model, per_example_lm_loss, clipping_norm=0.05, return_aux=True,
                                dtype=torch.float32)
    (out, aux), _ = fn(ids.to(dev), tgt.to(dev), state=st)
    for i, n in enumerate(names):
        assert _rel(out.pytree[n], res.reduced[i]) < 2e-2, n
    assert _rel(aux.grad_norms, res.norms) < 2e-2


@pytest.mark.parametrize("stream", ["reference", "device"])
def test_ghost_block_fused_noise_equals_separate_noise(dev, stream):
    torch.manual_seed(4)
    model = BlockLM(100, 64, 4, 96, dtype=torch.bfloat16).to(dev)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0.0, 0.05)
    g = torch.Generator().manual_seed(8)
    ids = torch.randint(0, 100, (3, 64), generator=g).to(dev)
    tgt = torch.randint(0, 100, (3, 64), generator=g).to(dev)
    names = sorted(n for n, p in model.named_parameters() if p.requires_grad)
    C = _groups(names)
    fn, st = ghost_clipped_grad(model, per_example_lm_loss, clipping_norm=C, normalize_by=2.0,
                                dtype=torch.float32)
    noise_fn, nstate = gaussian_noise(noise_multiplier=0.7, key=key(11), stream=stream)
    fused, _, _ = fn(ids, tgt, state=st, noise_fn=noise_fn, noise_state=nstate)
    plain, _ = fn(ids, tgt, state=st)
    separate, _ = noise_fn(plain, nstate)
    assert isinstance(fused, NoisedPytree)
    for n in names:
        assert torch.equal(fused.pytree[n], separate.pytree[n]), n


@pytest.mark.parametrize("per_group", [False, True])
def test_ghost_block_auto_s_matches_per_example_oracle(dev, per_group):
    # AUTO-S on the model path (auto_clipped_grad, _auto.py:211-367): scale
    # R / (||g|| + gamma) per example (per group), no min(1, .); the clipped
    # norms R ||g|| / (||g|| + gamma) stay below R (the DP bound).
    ref, ids, tgt = _case(torch.float32, 61, 32, 4, 48, 3, 20, seed=5)
    model = BlockLM(61, 32, 4, 48, dtype=torch.float32).to(dev)
    model.load_state_dict({k: v.float() for k, v in ref.state_dict().items()})
    names = sorted(n for n, p in model.named_parameters() if p.requires_grad)
    R = _groups(names) if per_group else 0.25
    res = _oracle(ref, ids, tgt, R, names, kind="auto_s", gamma=0.02)
    fn, st = auto_ghost_clipped_grad(model, per_example_lm_loss, R=R, gamma=0.02,
                                     normalize_by=3.0, return_aux=True)
    (out, aux), _ = fn(ids.to(dev), tgt.to(dev), state=st)
    assert out.max_norm == (R / 3.0 if not per_group else out.max_norm)
    for i, n in enumerate(names):
        assert _rel(out.pytree[n], res.reduced[i] / 3.0) < 1e-5, n
    torch.testing.assert_close(aux.clipped_grad_norms.cpu().double(),
                               res.clipped_norms.double(), rtol=1e-4, atol=1e-9)
    if per_group:
        for gname in ("attn", "mlp"):
            torch.testing.assert_close(aux.group_norms[gname].cpu().double(),
                                       res.group_norms[gname], rtol=1e-5, atol=0)
        parts = [aux.clip_scales[k][0].double() * aux.group_norms[g].double()
                 for k, g in enumerate(sorted(aux.group_norms))]
        bounds = [R.values[g] for g in sorted(aux.group_norms)]
        for part, bound in zip(parts, bounds):
            assert torch.all(part <= bound)
    else:
        torch.testing.assert_close(aux.grad_norms.cpu().double(), res.norms, rtol=1e-5, atol=0)
        assert torch.all(aux.clipped_grad_norms.double() <= R)
