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


# Widths % 4 != 0 take the general kernels.  In bfloat16, wide widths % 8 ==
# 0 with an even narrow width take the MFMA kernel: split chunks (2, 2048,
# 4096, 16), (3, 1000, 16, 1024) (a partial last step), an odd token count
# with a tail column block of 8 (1, 4097, 8, 520), one step written directly
# (8, 64, 14336, 16), 17..32 narrow columns with the narrow side the output
# (3, 96, 4096, 32) or the input (2, 512, 24, 2048), narrow widths 2 and 6
# (2, 333, 2, 1024), (1, 2100, 4104, 6) and a partial column block (2, 1056,
# 520, 8); the other widths % 4 == 0 the 8-wave v_dot2 kernel: (2, 130, 1,
# 700), an odd narrow width (1, 300, 1200, 17) and split chunks past one LDS
# chunk (2, 2500, 2044, 16).
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,din,dout", [(3, 77, 513, 16), (2, 64, 16, 1030), (4, 5, 32, 33),
                                          (2, 130, 1, 700), (1, 300, 1200, 17),
                                          (2, 2048, 4096, 16), (3, 1000, 16, 1024),
                                          (1, 4097, 8, 520), (8, 64, 14336, 16),
                                          (2, 512, 24, 2048), (3, 96, 4096, 32),
                                          (2, 1056, 520, 8), (2, 333, 2, 1024),
                                          (1, 2100, 4104, 6), (2, 2500, 2044, 16)])
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


# The grouped call: every problem as the oracle has it, whatever launch it
# lands in -- 37 bfloat16 problems (two MFMA launches of up to 24 in the
# 16-column class, one in the 32-column class; narrow side the input or the
# output), problems the MFMA kernel does not take (wide side % 8 != 0, an odd
# narrow side) run one by one, and the same set in float32 (none in MFMA
# launches).  Few workgroups (T = 300) make the launches split the tokens.
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T", [300, 64])
def test_per_example_grads_grouped_match_oracle(dev, dtype, T):
    B = 2
    g = torch.Generator().manual_seed(T)
    dims = [(96, 16), (16, 520), (24, 2048), (4096, 32), (1028, 12), (17, 600), (8, 8)]
    dims += [(64 + 8 * i, 2 + 2 * (i % 8)) for i in range(30)]
    A = [torch.randn(B, T, din, generator=g).to(dtype) for din, _ in dims]
    G = [torch.randn(B, T, dout, generator=g).to(dtype) for _, dout in dims]
    got = ops.per_example_grads_grouped([a.to(dev) for a in A], [x.to(dev) for x in G],
                                        out_dtype=torch.float32)
    got_bf = ops.per_example_grads_grouped([a.to(dev) for a in A], [x.to(dev) for x in G],
                                           out_dtype=torch.bfloat16)
    for k, (a, x) in enumerate(zip(A, G)):
        want = ghost_oracle.linear_per_example_grads(a, x, dtype=torch.float64)[0]
        assert got[k].shape == want.shape, k
        assert _rel(got[k], want) < 1e-5, k
        assert torch.equal(got_bf[k].cpu(), got[k].cpu().to(torch.bfloat16)), k


# Problems that share their wide operand (the same tensor) run as one group of
# the MFMA launch, up to three to a group: five narrow-output problems on one
# input x (widths 16, 2, 8, 14, 6: a group of three, then one of two), two
# narrow-input problems on one output gradient y, a problem whose wide side
# is x but as its output gradient (another output layout: not merged with
# x's), and one of narrow width 24 on x (the 32-column class: a launch of its
# own).  T = 300 splits the tokens, T = 2048 (B = 4) writes directly.
@pytest.mark.parametrize("B,T", [(2, 300), (4, 2048)])
def test_per_example_grads_grouped_shared_wide(dev, B, T):
    g = torch.Generator().manual_seed(T + B)
    bf = torch.bfloat16
    x = torch.randn(B, T, 1032, generator=g).to(bf)
    y = torch.randn(B, T, 520, generator=g).to(bf)
    narrow = {w: torch.randn(B, T, w, generator=g).to(bf) for w in (16, 2, 8, 14, 6, 12, 4, 24)}
    pairs = [(x, narrow[16]), (x, narrow[2]), (narrow[12], y), (x, narrow[8]),
             (narrow[4], x), (x, narrow[14]), (narrow[6], y), (x, narrow[6]), (x, narrow[24])]
    xd, yd = x.to(dev), y.to(dev)
    nd = {w: t.to(dev) for w, t in narrow.items()}

    def on_dev(t):
        return xd if t is x else yd if t is y else nd[t.shape[-1]]

    for out_dtype in (torch.float32, torch.bfloat16):
        got = ops.per_example_grads_grouped([on_dev(a) for a, _ in pairs],
                                            [on_dev(o) for _, o in pairs], out_dtype=out_dtype)
        for k, (a, o) in enumerate(pairs):
            want = ghost_oracle.linear_per_example_grads(a, o, dtype=torch.float64)[0]
            assert got[k].shape == want.shape, k
            if out_dtype == torch.float32:
                assert _rel(got[k], want) < 1e-5, k
            else:
                assert _rel(got[k], want) < 1e-2, k


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
    real = ops.per_example_grads_grouped
    monkeypatch.setattr(ops, "per_example_grads_grouped",
                        lambda A_list, G_list, **k: calls.extend(A_list) or real(A_list, G_list, **k))
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
