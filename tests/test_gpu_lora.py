"""GPU parity of the direct (materialised) per-example path: LoRA adapters.

Kernel level: ``per_example_grads`` (``dpc_per_example_grads``) against the
oracle's ``G_i^T A_i`` for narrow din or dout (1, 16, 17, 32), odd widths and
token counts, float32 and bfloat16.  Model level: ``ghost_clipped_grad`` on a
``LoRABlock`` (only the 14 adapters trainable; each takes the direct method)
against a loop of single-example backward passes clipped by the streaming
oracle.  Tolerances: 1e-5 relative (float32), 2e-2 relative (bfloat16).
"""

from __future__ import annotations

import pytest
import torch

from opake_amd import ops
from opake_amd.clipping import ghost_clipped_grad
from opake_amd.lora import LoRABlock
from opake_amd.noise import gaussian_noise
from opake_amd.random import key
from oracle import clip_oracle, ghost_oracle

pytestmark = pytest.mark.gpu


def _rel(got, want):
    got, want = got.double().cpu(), want.double().cpu()
    return ((got - want).norm() / want.norm().clamp_min(1e-300)).item()


# Widths % 4 != 0 take the general kernels; the others (bf16) the pipelined
# 8-wave kernel: split chunks (2, 2048, 4096, 16), (3, 1000, 16, 1024), an odd
# token count past one LDS chunk with a tail column block (1, 4097, 8, 520),
# one chunk written directly (8, 64, 14336, 16), 17..32 narrow columns with
# the narrow side the output (1, 300, 1200, 17), (3, 96, 4096, 32) or the
# input (2, 512, 24, 2048), and a partial column block (2, 1056, 520, 8).
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,din,dout", [(3, 77, 513, 16), (2, 64, 16, 1030), (4, 5, 32, 33),
                                          (2, 130, 1, 700), (1, 300, 1200, 17),
                                          (2, 2048, 4096, 16), (3, 1000, 16, 1024),
                                          (1, 4097, 8, 520), (8, 64, 14336, 16),
                                          (2, 512, 24, 2048), (3, 96, 4096, 32),
                                          (2, 1056, 520, 8)])
def test_per_example_grads_match_oracle(dev, dtype, B, T, din, dout):
    g = torch.Generator().manual_seed(B * 1000 + din + dout)
    A = torch.randn(B, T, din, generator=g).to(dtype)
    G = torch.randn(B, T, dout, generator=g).to(dtype)
    # The oracle sums the same (bf16-representable) inputs in float64; the
    # kernels form each product exactly and sum in float32.
    want = ghost_oracle.linear_per_example_grads(A, G, dtype=torch.float64)[0]
    got = ops.per_example_grads(A.to(dev), G.to(dev), out_dtype=torch.float32)
    assert got.shape == (B, dout, din)
    assert _rel(got, want) < 1e-5
    got_bf = ops.per_example_grads(A.to(dev), G.to(dev), out_dtype=torch.bfloat16)
    assert torch.equal(got_bf.cpu(), got.cpu().to(torch.bfloat16))
    # Deterministic: a second call gives the same bits.
    assert torch.equal(ops.per_example_grads(A.to(dev), G.to(dev), out_dtype=torch.float32), got)


def _case(dtype, seed=0):
    torch.manual_seed(seed)
    ref = LoRABlock(d=64, n_heads=4, n_kv_heads=2, ffn=96, r=4, dtype=torch.float64)
    with torch.no_grad():
        for p in ref.parameters():
            p.normal_(0.0, 0.1)
            if dtype == torch.bfloat16:
                p.copy_(p.to(torch.bfloat16).double())
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(3, 64, 64, generator=g)
    t = torch.randn(3, 64, 64, generator=g)
    if dtype == torch.bfloat16:
        x = x.to(torch.bfloat16)
    return ref, x, t


def _sq(out, t):
    return ((out.float() - t.float()) ** 2).sum(dim=(1, 2))


def _oracle(ref, x, t, C, names):
    per = ghost_oracle.per_example_grads_loop(ref, _sq, (x.double(),), t.double())
    leaves = [per[n].float() for n in names]
    return clip_oracle.stream_clip_and_sum(leaves, clip_oracle.conservative_bound(C))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ghost_lora_block_matches_per_example_oracle(dev, dtype, monkeypatch):
    ref, x, t = _case(dtype)
    model = LoRABlock(d=64, n_heads=4, n_kv_heads=2, ffn=96, r=4, dtype=dtype).to(dev)
    model.load_state_dict({k: v.to(dtype) for k, v in ref.state_dict().items()})
    names = sorted(n for n, p in model.named_parameters() if p.requires_grad)
    assert len(names) == 14
    calls = []
    real = ops.per_example_grads
    monkeypatch.setattr(ops, "per_example_grads",
                        lambda *a, **k: calls.append(1) or real(*a, **k))
    C = 0.5
    res = _oracle(ref, x, t, C, names)
    fn, st = ghost_clipped_grad(model, _sq, clipping_norm=C, normalize_by=2.0, return_aux=True,
                                dtype=torch.float32)
    (out, aux), _ = fn(x.to(dev), t.to(dev), state=st)
    assert len(calls) == 14  # every adapter took the direct method
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for i, n in enumerate(names):
        assert _rel(out.pytree[n], res.reduced[i] / 2.0) < tol, n
    assert _rel(aux.grad_norms, res.norms) < tol


def test_ghost_lora_fused_noise_equals_separate_noise(dev):
    ref, x, t = _case(torch.bfloat16, seed=3)
    model = LoRABlock(d=64, n_heads=4, n_kv_heads=2, ffn=96, r=4, dtype=torch.bfloat16).to(dev)
    model.load_state_dict({k: v.to(torch.bfloat16) for k, v in ref.state_dict().items()})
    fn, st = ghost_clipped_grad(model, _sq, clipping_norm=1.0, dtype=torch.float32)
    for stream in ("reference", "device"):
        noise_fn, nstate = gaussian_noise(noise_multiplier=1.1, key=key(2), stream=stream)
        fused, _, _ = fn(x.to(dev), t.to(dev), state=st, noise_fn=noise_fn, noise_state=nstate)
        plain, _ = fn(x.to(dev), t.to(dev), state=st)
        separate, _ = noise_fn(plain, nstate)
        for n in plain.pytree:
            assert torch.equal(fused.pytree[n], separate.pytree[n]), (stream, n)
