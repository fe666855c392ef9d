"""Correctness at the BASELINE sizes of the GPU configurations (GPU tests).

The smaller parity tests cover every code path on reduced shapes; these run
the exact launches the benchmark times -- config 2 (one linear layer 4096 x
4096, B = 32, T = 512, bf16: 256 output tiles, no split-K, the 8-way XCD
remap, an 8192-step K loop), config 3 (the Llama-style block, d = 2048, B =
16, T = 1024), config 4 (LoRA r = 16 on an 8B-shaped block, B = 8, T = 2048)
and config 5 (the top-2 MoE, 8 experts 2048 / 5632, B = 16, T = 1024) -- on
the benchmark's own synthetic inputs, and check them against float64
mathematics computed on the device:

* per-example squared norms against the exact ``||G_i^T A_i||^2`` (fp64
  Gram identity), 2e-2 relative (observed ~1e-4), and inside the returned
  error bound;
* clip scales bit-exact against the host float64 evaluation of the
  reference's guarded ratio from the device's norm and bound (config 2), and
  the DP bound ``scale_i ||G_i^T A_i|| <= C`` with no tolerance;
* sampled output rows of every clipped sum (all columns) against the float64
  sum ``sum_i scale_i G_i[:, m]^T A_i`` with the device's scales, 1e-5
  relative (fp32 accumulation);
* config 3's block norm from the multi-layer Gram launch, both sides, against
  the exact projection norms plus the RMSNorm weights' per-example squares;
* config 4's grouped per-example gradients (16 sampled rows of every adapter
  and example) against float64 at 1e-5, the bf16 launch equal to the fp32
  one rounded, the leaf clip-and-sum against float64 with the device's
  scales, and the fused noise equal to ``noise_fn`` on the noiseless result;
* at config 2, the fused noise: an injected float32 draw is added bit-exactly
  (``to_bf16(v + sigma z)``), and the Philox epilogue equals ``dpc_add_noise``
  on the noiseless output.
"""

from __future__ import annotations

import math

import pytest
import torch

import bench
from opake_amd import _native as nat
from opake_amd import ops
from opake_amd.clipping import (ghost_capture, ghost_clip_captured, ghost_clip_sum,
                                guard_for_linear)
from opake_amd.clipping import _numerics as num
from opake_amd.clipping._model import LinearCapture
from opake_amd.transformer import per_example_lm_loss
from oracle import clip_oracle

pytestmark = pytest.mark.gpu


def _gram64(X):
    """[B, T, d] -> [B, T, T] float64 Gram matrices on the device."""
    X = X.double()
    return torch.matmul(X, X.transpose(1, 2).contiguous())


def _exact_sqnorms(A, G):
    """||G_i^T A_i||^2 per example, float64 on the device (Gram identity)."""
    out = torch.empty(A.shape[0], dtype=torch.float64, device=A.device)
    for i in range(A.shape[0]):  # one example at a time bounds the fp64 memory
        out[i] = (_gram64(A[i:i + 1]) * _gram64(G[i:i + 1])).sum()
    return out


def _rows_exact(A, G, scale, rows):
    """Rows ``rows`` of sum_i scale_i G_i^T A_i in float64: [len(rows), din]."""
    B, T = A.shape[0], A.shape[1]
    g = (G[:, :, rows].double() * scale.double().view(B, 1, 1)).reshape(B * T, len(rows))
    return g.t() @ A.reshape(B * T, -1).double()


def _rel(got, want):
    got, want = got.double(), want.double()
    return ((got - want).norm() / want.norm().clamp_min(1e-300)).item()


def _sample_rows(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(n, generator=g)[:k].sort().values.tolist()


# --- config 2 ---------------------------------------------------------------------


@pytest.fixture(scope="module")
def cfg2(dev):
    A, G = bench.make_inputs(dev)
    return A, G


def test_cfg2_norms_scales_and_bound(dev, cfg2):
    A, G = cfg2
    B, T, din = A.shape
    dout = G.shape[2]
    sq, err = ops.gram_sqnorms(A, G, return_error=True)
    exact = _exact_sqnorms(A, G)
    assert torch.all((sq - exact).abs() <= err)
    assert torch.all((sq - exact).abs() / exact < 2e-2)
    assert torch.all(err / sq < 2e-2)
    # Clip scales: the device against the host float64 evaluation of the same
    # formula (guarded ratio of C over sqrt(sq + err)).
    C = num.conservative_bound(bench.C)
    guard = guard_for_linear(A.dtype, din, dout, False)
    cf = ops.clip_factors(sq, C, [guard], err=err, count_threshold=num.float32_of(bench.C))
    up = (sq + err).cpu()
    up = torch.where(up < 0, torch.zeros_like(up), up)
    roundoff = num.norm_roundoff(torch.float32, torch.float64, 1,
                                 num.reduction_terms([din * dout]))
    want = clip_oracle.finalize_scale(C / torch.sqrt(up), A.dtype, torch.float32, roundoff,
                                      clamp_to_one=True).to(torch.float32)
    assert torch.equal(cf.scale[0].cpu(), want)
    # DP bound, no tolerance; clip decisions away from the boundary.
    s = cf.scale[0].double()
    assert torch.all(s * exact.sqrt() <= bench.C)
    norms = exact.sqrt()
    away = ((norms - bench.C).abs() / bench.C > 1e-3)
    assert int(cf.nclipped.item()) == int(((cf.norms.double() > bench.C)).sum().item())
    assert torch.equal((cf.norms.double() > bench.C)[away], (norms > bench.C)[away])
    assert 8 <= int(cf.nclipped.item()) <= 24  # about half of 32 are clipped


def test_cfg2_clipped_sum_sampled_rows(dev, cfg2):
    A, G = cfg2
    res, aux = ghost_clip_sum(A, G, clipping_norm=bench.C, return_aux=True,
                              dtype=torch.float32)
    w = res.pytree["weight"]
    assert w.shape == (G.shape[2], A.shape[2]) and torch.isfinite(w).all()
    rows = _sample_rows(G.shape[2], 64, 0)
    want = _rows_exact(A, G, aux.clip_scales, rows)
    assert _rel(w[rows], want) < 1e-5
    # bf16 output (the benchmark's): the fp32 sum rounded once.
    res16 = ghost_clip_sum(A, G, clipping_norm=bench.C)
    w16 = res16.pytree["weight"]
    assert w16.dtype == torch.bfloat16
    assert torch.equal(w16, w.to(torch.bfloat16))


def test_cfg2_noise_epilogues(dev, cfg2):
    A, G = cfg2
    B, T, din = A.shape
    dout = G.shape[2]
    sq, err = ops.gram_sqnorms(A, G, return_error=True)
    cf = ops.clip_factors(sq, num.conservative_bound(bench.C),
                          [guard_for_linear(A.dtype, din, dout, False)], err=err,
                          count_threshold=1.0)
    center, _ = ops.clipped_sum(A, G, cf.scale[0], plan=cf.plan[0])
    sigma = bench.NM * bench.C
    # Injected draw: to_bf16(float(v) + float32(sigma) * z), bit for bit.
    z = torch.randn(dout, din, generator=torch.Generator(device=dev).manual_seed(5), device=dev)
    spec = ops.NoiseSpec(sigma=sigma, mode=nat.NOISE_INJECTED, noise=z)
    noisy, _ = ops.clipped_sum(A, G, cf.scale[0], plan=cf.plan[0], noise=spec)
    s32 = torch.tensor(sigma, dtype=torch.float32, device=dev)
    assert torch.equal(noisy, (center.float() + s32 * z).to(torch.bfloat16))
    # Philox: the fused epilogue draws the same stream as the noise kernel.
    spec = ops.NoiseSpec(sigma=sigma, mode=nat.NOISE_PHILOX, seed=0x1234_5678_9ABC, leaf_id=0)
    fused, _ = ops.clipped_sum(A, G, cf.scale[0], plan=cf.plan[0], noise=spec)
    sep = ops.add_noise(center, sigma, mode=nat.NOISE_PHILOX, seed=0x1234_5678_9ABC, leaf_id=0)
    assert torch.equal(fused, sep)


# --- config 3 ---------------------------------------------------------------------


def test_cfg3_block_projections(dev):
    model = bench.block_model(dev, torch.bfloat16)
    g = torch.Generator(device=dev).manual_seed(0)
    ids = torch.randint(0, bench.BLK_V, (bench.BLK_B, bench.BLK_T), generator=g, device=dev)
    tgt = torch.randint(0, bench.BLK_V, (bench.BLK_B, bench.BLK_T), generator=g, device=dev)
    caps, _ = ghost_capture(model, per_example_lm_loss, ids, tgt)
    linears = [c for c in caps if isinstance(c, LinearCapture)]
    assert len(linears) == 4
    total_exact = torch.zeros(bench.BLK_B, dtype=torch.float64, device=dev)
    for c in linears:
        sq, err = ops.gram_sqnorms(c.A, c.G, return_error=True)
        exact = _exact_sqnorms(c.A, c.G)
        total_exact += exact
        assert torch.all((sq - exact).abs() <= err), c.name
        assert torch.all((sq - exact).abs() / exact < 2e-2), c.name
    res, aux = ghost_clip_captured(caps, clipping_norm=bench.C, return_aux=True,
                                   dtype=torch.float32)
    scale = aux.clip_scales[0]
    for k, c in enumerate(linears):
        w = res.pytree[f"{c.name}.weight"]
        rows = _sample_rows(c.G.shape[2], 16, k)
        assert _rel(w[rows], _rows_exact(c.A, c.G, scale, rows)) < 1e-5, c.name
    # The block's norm, from the multi-layer Gram launch the benchmark times
    # (dpc_gram_sqnorms_multi) plus the leaf kernels: the projections' exact
    # squared norms plus the RMSNorm weights' materialised per-example
    # gradients, both sides.
    direct = [c for c in caps if not isinstance(c, LinearCapture)]
    assert len(direct) == 1
    for g in direct[0].grads.values():
        total_exact += g.double().reshape(g.shape[0], -1).square().sum(dim=1)
    got = aux.grad_norms.double() ** 2
    assert torch.all((got - total_exact).abs() / total_exact < 2e-2), got / total_exact
    assert torch.all(scale.double() * total_exact.sqrt() <= bench.C)


# --- config 4 ---------------------------------------------------------------------


def test_cfg4_lora_block(dev):
    """The launches config 4 times: all 14 adapter sides' per-example
    gradients in one grouped launch (narrow_wide_mfma_kernel over the 11
    shared-wide groups: wide sides 4096 and 14336, B = 8, T = 2048), then the
    leaf clip-and-sum and the fused Philox noise."""
    from opake_amd.noise import gaussian_noise
    from opake_amd.random import key

    model = bench.lora_model(dev, torch.bfloat16)
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(bench.LORA_B, bench.LORA_T, bench.LORA_D, generator=g,
                    device=dev).to(torch.bfloat16)
    tgt = torch.randn(bench.LORA_B, bench.LORA_T, bench.LORA_D, generator=g, device=dev)
    caps, _ = ghost_capture(model, bench._mse_loss, x, tgt)
    linears = [c for c in caps if isinstance(c, LinearCapture)]
    assert len(linears) == 14 and all(min(c.A.shape[-1], c.G.shape[-1]) <= 16 for c in linears)
    B = bench.LORA_B
    # The model path's grouped launch, its operands as the model path forms them.
    As = [c.A.reshape(B, -1, c.A.shape[-1]) for c in linears]
    Gs = [c.G.reshape(B, -1, c.G.shape[-1]) for c in linears]
    g32 = ops.per_example_grads_grouped(As, Gs, out_dtype=torch.float32)
    g16 = ops.per_example_grads_grouped(As, Gs)
    exact_sq = torch.zeros(B, dtype=torch.float64, device=dev)
    for k, (c, A, G, w32, w16) in enumerate(zip(linears, As, Gs, g32, g16)):
        rows = _sample_rows(G.shape[2], 16, k)
        for b in range(B):
            want = G[b][:, rows].double().t() @ A[b].double()
            assert _rel(w32[b][rows], want) < 1e-5, (c.name, b)
        # The bf16 launch stores the same fp32 sums, rounded.
        assert torch.equal(w16, w32.to(torch.bfloat16)), c.name
        exact_sq += w16.double().reshape(B, -1).square().sum(dim=1)
    # Clip and sum (leaf kernels) against float64 with the device's scales.
    res, aux = ghost_clip_captured(caps, clipping_norm=bench.C, return_aux=True,
                                   dtype=torch.float32)
    got = aux.grad_norms.double() ** 2
    assert torch.all((got - exact_sq).abs() / exact_sq < 1e-5), got / exact_sq
    scale = aux.clip_scales[0]
    for c, w16 in zip(linears, g16):
        stored = (w16.float() * scale.view(B, 1, 1)).to(torch.bfloat16)
        want = stored.double().sum(dim=0)
        assert _rel(res.pytree[f"{c.name}.weight"], want) < 1e-5, c.name
    # Every example's stored gradient is within C (the guard covers the bf16 store).
    stored_sq = torch.zeros(B, dtype=torch.float64, device=dev)
    for w16 in g16:
        st = (w16.float() * scale.view(B, 1, 1)).to(torch.bfloat16).double()
        stored_sq += st.reshape(B, -1).square().sum(dim=1)
    assert torch.all(stored_sq.sqrt() <= bench.C)
    # The fused Philox noise equals noise_fn on the noiseless result, bit for bit.
    noise_fn, state = gaussian_noise(noise_multiplier=bench.NM, key=key(0), stream="device")
    noised, _ = ghost_clip_captured(caps, clipping_norm=bench.C, noise_fn=noise_fn,
                                    noise_state=state)
    plain = ghost_clip_captured(caps, clipping_norm=bench.C)
    separate, _ = noise_fn(plain, state)
    assert set(noised.pytree) == set(separate.pytree)
    for n in noised.pytree:
        assert torch.equal(noised.pytree[n], separate.pytree[n]), n


# --- config 5 ---------------------------------------------------------------------


def test_cfg5_moe_grouped(dev):
    caps, counts = bench.moe_captures(dev)
    pg = bench.moe_groups()
    res, aux = ghost_clip_captured(caps, clipping_norm=pg, return_aux=True, dtype=torch.float32)
    E, Bm = counts.shape
    group_names = sorted(pg.values)
    for e in range(E):
        seg = counts[e].tolist()
        starts = [0]
        for n in seg:
            starts.append(starts[-1] + n)
        pair = [c for c in caps if c.name.startswith(f"experts.{e}.")]
        # Per-example per-expert squared norms (both projections), exact.
        exact = torch.zeros(Bm, dtype=torch.float64, device=dev)
        for c in pair:
            for b in range(Bm):
                if seg[b]:
                    a = c.A[starts[b]:starts[b + 1]].unsqueeze(0)
                    gg = c.G[starts[b]:starts[b + 1]].unsqueeze(0)
                    exact[b] += (_gram64(a) * _gram64(gg)).sum()
        got = aux.group_norms[group_names[e]].double()
        nz = exact > 0
        assert torch.all((got[nz] ** 2 - exact[nz]).abs() / exact[nz] < 2e-2), e
        scale = aux.clip_scales[e][0] if aux.clip_scales.dim() == 3 else aux.clip_scales[e]
        c_e = pg.values[group_names[e]]
        assert torch.all(scale.double() * exact.sqrt() <= c_e), e
        for c in pair:
            w = res.pytree[f"{c.name}.weight"]
            rows = _sample_rows(c.G.shape[1], 8, e)
            seg_scale = torch.repeat_interleave(scale.double(), counts[e].to(dev))
            g = c.G[:, rows].double() * seg_scale.unsqueeze(1)
            want = g.t() @ c.A.double()
            assert _rel(w[rows], want) < 1e-5, c.name
