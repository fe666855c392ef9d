"""DP-SGD clip -> sum -> noise step throughput on one MI355X.

Workload: one sequence linear layer, d_in = d_out = 4096,
bf16 activations A [B=32, T=512, 4096] ~ N(0, 1) and output gradients G of the
same batch/sequence shape.  G is N(0, sigma_G) with sigma_G = C / sqrt(T * d_in
* d_out) and each example scaled by a lognormal(0, 1) factor, so that about half
of the examples are clipped (at the configuration's literal N(0, 1e-2) every
example would be clipped by ~900x).  C = 1.0, noise multiplier 1.0,
normalize_by = 1 (the reference default), noise from the device (Philox)
stream fused into the clipped-sum epilogue.

A step is one ``ghost_clip_sum`` call: Gram norms -> clip factors -> clipped-sum
GEMM with the fused noise epilogue, inputs resident in HBM.  The timed region
is bracketed by ``torch.cuda.synchronize()``.  The dominant kernel (the
clipped-sum GEMM) is timed with HIP events recorded on the stream it is
launched on, inside the timed steps.

``cpu_baseline``: the reference algorithm restated on the CPU (``vmap(grad)``
of the linear surrogate loss, the streaming clip-and-sum, the CPU-generator
noise draw) on a bounded sample of the same workload: the full layer with a
reduced batch, timed on the host cores of the box.

``--config 1`` measures BASELINE configs[0], the reference's CPU-runnable
MLP (784-512-10, fp32, B = 256): the whole DP step on the GPU, eagerly and with
the clip part replayed from a HIP graph; ``cpu_baseline`` there is the full
configuration on the CPU.

``--config 3`` (not the default line) measures BASELINE configs[2]: a
Llama-style block (d = 2048, 16 heads, SwiGLU 8192, RMSNorm, RoPE, bf16, B =
16, T = 1024, vocab 32000, embedding and head frozen); ``value`` is the ghost
clip -> sum -> noise of the block's parameters from one step's captured
operands, and ``config.full_step_ms`` the whole step with the forward and the
backward to the module outputs on PyTorch-ROCm.

``--config 4`` measures BASELINE configs[3]: LoRA r = 16 adapters on the seven
projections of an 8B-shaped block, B = 8, T = 2048, bf16; the adapters'
per-example gradients are formed directly (the Gram norm would cost 64x
more), then clipped, summed and noised as materialised leaves; the roofline
is HBM bandwidth of the per-example gradient kernel.

``--config 5`` (not the default line) measures BASELINE configs[4] the same
way: a top-2 MoE FFN with 8 SwiGLU experts (d = 2048, expert width 5632),
bf16, B = 16, T = 1024, routing from N(0, 1) router logits; the step is the
per-expert ghost clipping of the 16 expert projections from their captured
inputs and output gradients (grouped Gram norms, per-expert clip factors with
C_e = C / sqrt(8), grouped clipped-sum GEMMs with per-group noise fused), the
model's forward and backward excluded.

``--path leaves`` (config 2, not the default line) runs the materialised-leaf
path -- the reference's own streaming clip-and-sum as the fused-backend seam
runs it -- over the config-2 layer's per-example gradients ([32, 4096, 4096]
bf16, synthetic, resident in HBM) and times each pass on its own (norm pass,
clip factors, scale-store-sum pass, device-stream noise pass) with its bytes
and GB/s against the HBM peak.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import opake_amd  # noqa: E402,F401  (first: it sets HIP's options before the GPU is used)
import torch  # noqa: E402,F401  (every measured path needs it)

METRIC = "DP-step examples/sec at 1 MI355X; TFLOP/s and % of MFMA/HBM roofline"
B, T, DIN, DOUT = 32, 512, 4096, 4096
C, NM = 1.0, 1.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBS = 8000.0
CLOCK_SETTLE_S = 0.2  # untimed steps before the warm-up of the default line


def algorithmic_flops(b=B, t=T, din=DIN, dout=DOUT):
    """Gram norms (SYRK convention T(T+1)(din+dout)), inner products 2T^2, GEMM 2BTdin dout."""
    gram = b * (t * (t + 1) * (din + dout) + 2 * t * t)
    gemm = 2 * b * t * din * dout
    return gram, gemm


def make_inputs(device, b=B, t=T, din=DIN, dout=DOUT, seed=0):
    import torch

    g = torch.Generator(device=device).manual_seed(seed)
    A = torch.randn(b, t, din, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    sigma_g = C / math.sqrt(t * din * dout)
    lognormal = torch.exp(torch.randn(b, 1, 1, generator=g, device=device))
    G = (torch.randn(b, t, dout, generator=g, device=device) * sigma_g * lognormal).to(
        torch.bfloat16)
    return A, G


CPU_REPEATS = 5  # timed CPU-baseline steps (median) after one warm-up


def cpu_threads() -> int:
    """Host threads for the CPU baseline: every CPU this process may run on,
    capped by OMP_NUM_THREADS when the environment sets it (the GPU box sets
    it to the host share of one GPU)."""
    visible = len(os.sched_getaffinity(0))
    try:
        share = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        share = 0
    return min(visible, share) if share > 0 else visible


def cpu_host() -> str:
    """CPU model and the CPUs visible to the process, for the baseline line."""
    return f"{cpu_model()}; {len(os.sched_getaffinity(0))} CPUs visible"


def median_rate(step, examples: int, repeats: int = CPU_REPEATS) -> float:
    """Examples/s of ``step`` (``examples`` per call): one warm-up call, then
    the median of ``repeats`` timed calls."""
    step()
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    return examples / times[len(times) // 2]


def cpu_baseline(sample_b: int, threads: int):
    """Reference restatement on the CPU (oracle package), examples/s."""
    import torch

    from oracle import clip_oracle, ghost_oracle, noise_oracle

    torch.set_num_threads(threads)
    A, G = make_inputs(torch.device("cpu"), b=sample_b, seed=1)

    def step():
        leaves = [ghost_oracle.surrogate_per_example_grads(A, G)]
        res = clip_oracle.stream_clip_and_sum(leaves, clip_oracle.conservative_bound(C))
        center = clip_oracle.normalize(res.reduced[0], 1.0)
        seed = noise_oracle.step_seed(0, 0)
        draw = noise_oracle.draws_for([center], seed)[0]
        return noise_oracle.sample(center, NM * C, draw)

    return median_rate(step, sample_b)


def measured_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed counter summary
    (FETCH_SIZE / WRITE_SIZE runs scaled by a copy-kernel calibration), or None."""
    path = os.path.join(ROOT, "profiles", "clipped_sum_cfg2_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(f"traffic_bytes_per_launch {kernel}:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def sustained_mfma_tflops(device, iters: int = 16384) -> float:
    """bf16 MFMA throughput the chip sustains on random N(0, 1) operands,
    measured with dpc_calib_mfma_bf16 (2 workgroups of 8 waves per CU running
    only back-to-back 32x32x16 MFMAs; best of 3 launches after 2 warm-ups).
    The published 2.5 PFLOP/s holds for operands that barely toggle; this is
    the ceiling a GEMM on real data can approach."""
    import torch

    from opake_amd import _native as nat

    grid = 2 * torch.cuda.get_device_properties(device).multi_processor_count
    ops_bytes = grid * 512 * 128
    operands = torch.randn(ops_bytes // 2, device=device).to(torch.bfloat16)
    out = torch.empty(grid * 512, device=device)
    stream = nat.stream_handle(device)
    times = []
    for rep in range(5):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        nat.call("dpc_calib_mfma_bf16", nat.ptr(operands), grid, iters, nat.ptr(out), stream)
        b.record()
        b.synchronize()
        if rep >= 2:
            times.append(a.elapsed_time(b) * 1e-3)
    flops = grid * 8 * iters * 8 * 2 * 32 * 32 * 16
    return flops / min(times) / 1e12


SUSTAINED_METHOD = ("dpc_calib_mfma_bf16 in this run: random N(0,1) bf16 operands, 2 "
                    "workgroups of 8 waves per CU, back-to-back 32x32x16 MFMAs (best of 3 "
                    "launches); context only, the roofline fraction is against `peak`")


def add_sustained(roofline: dict, device, sustained: float | None = None) -> dict:
    """Adds the measured sustained bf16 MFMA rate to a bf16 MFMA roofline as
    context (``frac`` stays against the published peak)."""
    if roofline.get("bound") == "mfma" and roofline.get("peak") == MFMA_BF16_PEAK_TFLOPS:
        roofline["sustained_mfma_tflops"] = (sustained if sustained is not None
                                             else sustained_mfma_tflops(device))
        roofline["sustained_method"] = SUSTAINED_METHOD
    return roofline


def library_reference(A, G, reps: int = 10) -> dict:
    """Same-box library time of the identical GEMM: sum over the B*T rows of
    G^T A (bf16 in, bf16 out, fp32 accumulation, no scales, no epilogue) by
    ``torch.mm`` (hipBLASLt / rocBLAS on ROCm), median of ``reps`` launches
    after 3 warm-ups -- in the operands' own layout (m- and n-contiguous rows,
    the reduction dimension slow) and with K-contiguous copies of both."""
    import torch

    rows = A.shape[0] * A.shape[1]
    din, dout = A.shape[2], G.shape[2]
    G2, A2 = G.reshape(rows, dout), A.reshape(rows, din)

    def median_ms(fn):
        for _ in range(3):
            fn()
        times = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            times.append(a.elapsed_time(b))
        times.sort()
        return times[len(times) // 2]

    natural = median_ms(lambda: torch.mm(G2.t(), A2))
    Gt, At = G2.t().contiguous(), A2.t().contiguous()
    kcontig = median_ms(lambda: torch.mm(Gt, At.t()))
    del Gt, At
    flops = 2.0 * rows * din * dout
    return {
        "op": "torch.mm (hipBLASLt): G^T A over B*T rows, bf16 -> bf16, fp32 accumulation",
        "natural_layout_ms": natural,
        "natural_layout_tflops": flops / (natural * 1e-3) / 1e12,
        "k_contiguous_copies_ms": kcontig,
        "k_contiguous_copies_tflops": flops / (kcontig * 1e-3) / 1e12,
    }


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


MOE_B, MOE_T, MOE_D, MOE_I, MOE_E, MOE_K = 16, 1024, 2048, 5632, 8, 2


def moe_captures(device, b=MOE_B, t=MOE_T, seed=0):
    """Captured operands of the config-5 expert projections, in the routed
    (expert-sorted, example-major) row layout, and the [E, b] row counts.

    Output gradients are N(0, sigma) with sigma chosen so that a segment of
    the mean length (t * k / E rows) has per-expert norm C_e, times a
    lognormal(0, 1) factor per example: about half of the (example, expert)
    groups are clipped."""
    import torch

    from opake_amd.clipping import LinearCapture

    g = torch.Generator(device=device).manual_seed(seed)
    logits = torch.randn(b, t, MOE_E, generator=g, device=device)
    expert = torch.topk(logits, MOE_K, dim=-1).indices.reshape(-1)
    token = torch.arange(b * t, device=device).repeat_interleave(MOE_K)
    counts = torch.bincount(expert * b + token // t, minlength=MOE_E * b).view(MOE_E, b).cpu()
    c_e = C / math.sqrt(MOE_E)
    mean_rows = t * MOE_K / MOE_E
    sigma = c_e / math.sqrt(mean_rows * (MOE_D * 2 * MOE_I + MOE_I * MOE_D))
    factor = torch.exp(torch.randn(b, generator=g, device=device))
    caps = []
    for e in range(MOE_E):
        seg = counts[e].tolist()
        n = sum(seg)
        row_f = torch.repeat_interleave(factor, counts[e].to(device)).unsqueeze(1) * sigma

        def rnd(cols, scale=None):
            x = torch.randn(n, cols, generator=g, device=device)
            return (x if scale is None else x * scale).to(torch.bfloat16)

        caps.append(LinearCapture(f"experts.{e}.gate_up", rnd(MOE_D), rnd(2 * MOE_I, row_f),
                                  segments=seg))
        caps.append(LinearCapture(f"experts.{e}.down", rnd(MOE_I), rnd(MOE_D, row_f),
                                  segments=seg))
    return caps, counts


def moe_groups():
    from opake_amd.types import PerGroup

    groups = {f"experts.{e}.{p}.weight": f"expert{e}" for e in range(MOE_E)
              for p in ("gate_up", "down")}
    return PerGroup(groups, {f"expert{e}": C / math.sqrt(MOE_E) for e in range(MOE_E)})


def moe_flops(counts):
    """Grouped Gram (SYRK convention per segment) and grouped clipped-sum FLOPs."""
    shapes = [(MOE_D, 2 * MOE_I), (MOE_I, MOE_D)]
    gram = gemm = 0
    for n in counts.reshape(-1).tolist():
        for din, dout in shapes:
            gram += n * (n + 1) * (din + dout) + 2 * n * n
            gemm += 2 * n * din * dout
    return gram, gemm


def moe_cpu_baseline(threads: int):
    """One example of the config-5 step on the CPU: per-expert gradients of the
    example materialised (its segment of each expert), the per-group streaming
    clip-and-sum and the CPU-generator noise.  Examples/s."""
    import torch

    from oracle import clip_oracle, ghost_oracle, noise_oracle

    torch.set_num_threads(threads)
    caps, counts = moe_captures(torch.device("cpu"), b=1, seed=1)
    pg = moe_groups()
    names = sorted(f"{c.name}.weight" for c in caps)
    by_name = {f"{c.name}.weight": c for c in caps}

    def step():
        leaves = []
        for n in names:
            c = by_name[n]
            leaves.append(ghost_oracle.segment_grads(c.A, c.G, c.segments, dtype=torch.bfloat16))
        groups = [pg.groups[(n,)] for n in names]
        values = {k: clip_oracle.conservative_bound(v) for k, v in pg.values.items()}
        res = clip_oracle.stream_clip_and_sum(leaves, None, groups=groups, group_values=values)
        seed = noise_oracle.step_seed(0, 0)
        draws = noise_oracle.draws_for(res.reduced, seed)
        sig = NM * math.sqrt(C / math.sqrt(MOE_E) * C * math.sqrt(MOE_E))
        return [noise_oracle.sample(x, sig, z) for x, z in zip(res.reduced, draws)]

    return median_rate(step, 1)


def run_moe(args) -> dict:
    import torch

    from opake_amd import _native
    from opake_amd.clipping import ghost_clip_captured
    from opake_amd.noise import gaussian_noise
    from opake_amd.random import key

    _native.load()
    dev = torch.device("cuda:0")
    caps, counts = moe_captures(dev)
    pg = moe_groups()
    noise_fn, state = gaussian_noise(noise_multiplier=NM, key=key(0), stream="device")

    def step(st, record):
        (res, aux), st = ghost_clip_captured(caps, clipping_norm=pg, noise_fn=noise_fn,
                                             noise_state=st, return_aux=True, gemm_events=record)
        return aux, st

    warm = max(1, args.warmup // 8)
    for _ in range(warm):
        aux, state = step(state, None)
    torch.cuda.synchronize()
    clipped_frac = int(aux.num_clipped.sum().item()) / (MOE_B * MOE_E)
    print(f"[bench] warmup done, clipped fraction {clipped_frac:.3f}", file=sys.stderr, flush=True)
    steps = max(1, args.steps // 8)
    events = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        aux, state = step(state, events)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    print(f"[bench] {steps} timed steps in {elapsed:.4f} s", file=sys.stderr, flush=True)
    gemm_ms = sum(a.elapsed_time(b) for a, b in events) / steps  # both launches of a step
    gram_f, gemm_f = moe_flops(counts)
    ms_per_step = 1e3 * elapsed / steps
    step_tflops = (gram_f + gemm_f) / (ms_per_step * 1e-3) / 1e12
    gemm_tflops = gemm_f / (gemm_ms * 1e-3) / 1e12
    cpu = None
    if not args.no_cpu_baseline:
        threads = cpu_threads()
        print(f"[bench] cpu baseline: 1 example on {threads} threads", file=sys.stderr, flush=True)
        cpu = {
            "value": moe_cpu_baseline(threads),
            "unit": "examples/s",
            "cores": threads,
            "kind": "port",
            "sample": ("config 5 at B=1: the example's per-expert gradients materialised from "
                       "its captured segments (16 leaves, 276.8M parameters), per-group "
                       f"streaming clip-and-sum, CPU randn noise; median of {CPU_REPEATS} steps after 1 "
                       f"warm-up; {cpu_host()}"),
        }
    return {
        "steps": steps,
        "warmup": warm,
        "ms_per_step": ms_per_step,
        "value": MOE_B * steps / elapsed,
        "config": {
            "workload": "top-2 MoE FFN, 8 SwiGLU experts d=2048 / 5632, B=16, T=1024, bf16; "
                        "per-expert ghost clipping of the expert projections from captured "
                        "operands + fused per-group device-stream noise (BASELINE configs[4])",
            "global_batch": MOE_B,
            "seq_len": MOE_T,
            "clipping_norm": "PerGroup C/sqrt(8) per expert",
            "noise_multiplier": NM,
            "normalize_by": 1.0,
            "routing": "top-2 of N(0,1) router logits (router frozen)",
            "clipped_fraction": clipped_frac,
            "step_tflops": step_tflops,
            "step_frac_of_bf16_peak": step_tflops / MFMA_BF16_PEAK_TFLOPS,
            "excluded": "model forward/backward (PyTorch-ROCm)",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "clipped_sum_bf16_kernel<true, false> (grouped; 2 grouped GEMMs per step, "
                      "one launch each)",
            "achieved": gemm_tflops,
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": gemm_tflops / MFMA_BF16_PEAK_TFLOPS,
            "avg_launch_ms": gemm_ms / 2,
            "traffic": None,
        },
        "cpu_baseline": cpu,
    }


BLK_B, BLK_T, BLK_D, BLK_H, BLK_F, BLK_V = 16, 1024, 2048, 16, 8192, 32000


def block_model(device, dtype, seed=0):
    import torch

    from opake_amd.transformer import BlockLM

    torch.manual_seed(seed)
    model = BlockLM(BLK_V, BLK_D, BLK_H, BLK_F, dtype=dtype, device=device)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0.0, 0.02)
    return model


def block_flops(b=BLK_B, t=BLK_T):
    """Gram norms (SYRK convention) and clipped-sum FLOPs of the block's four
    projections (qkv d->3d, o d->d, gate_up d->2F, down F->d)."""
    shapes = [(BLK_D, 3 * BLK_D), (BLK_D, BLK_D), (BLK_D, 2 * BLK_F), (BLK_F, BLK_D)]
    gram = b * sum(t * (t + 1) * (din + dout) + 2 * t * t for din, dout in shapes)
    gemm = b * sum(2 * t * din * dout for din, dout in shapes)
    return gram, gemm


def block_cpu_baseline(threads: int):
    """One example of the config-3 step on the CPU: per-example gradients of
    the block's parameters (forward and backward of the example alone), the
    streaming clip-and-sum and the CPU-generator noise.  Examples/s."""
    import torch

    from opake_amd.transformer import per_example_lm_loss
    from oracle import clip_oracle, ghost_oracle, noise_oracle

    torch.set_num_threads(threads)
    model = block_model(torch.device("cpu"), torch.float32, seed=1)
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, BLK_V, (1, BLK_T), generator=g)
    tgt = torch.randint(0, BLK_V, (1, BLK_T), generator=g)

    def step():
        per = ghost_oracle.per_example_grads_loop(model, per_example_lm_loss, (ids,), tgt)
        names = sorted(per)
        res = clip_oracle.stream_clip_and_sum([per[n] for n in names],
                                              clip_oracle.conservative_bound(C))
        draws = noise_oracle.draws_for(res.reduced, noise_oracle.step_seed(0, 0))
        return [noise_oracle.sample(x, NM * C, z) for x, z in zip(res.reduced, draws)]

    return median_rate(step, 1)


def run_block(args) -> dict:
    import torch

    from opake_amd import _native
    from opake_amd.clipping import ghost_capture, ghost_clip_captured, ghost_clipped_grad
    from opake_amd.noise import gaussian_noise
    from opake_amd.random import key
    from opake_amd.transformer import per_example_lm_loss

    _native.load()
    dev = torch.device("cuda:0")
    model = block_model(dev, torch.bfloat16)
    g = torch.Generator(device=dev).manual_seed(0)
    ids = torch.randint(0, BLK_V, (BLK_B, BLK_T), generator=g, device=dev)
    tgt = torch.randint(0, BLK_V, (BLK_B, BLK_T), generator=g, device=dev)
    noise_fn, state = gaussian_noise(noise_multiplier=NM, key=key(0), stream="device")

    # Full step: forward, backward to the module outputs, clip + sum + noise.
    fn, st = ghost_clipped_grad(model, per_example_lm_loss, clipping_norm=C, return_aux=True)
    full_steps = max(1, args.steps // 20)
    for _ in range(max(1, args.warmup // 40)):
        (_, aux), _, state = fn(ids, tgt, state=st, noise_fn=noise_fn, noise_state=state)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(full_steps):
        (_, aux), _, state = fn(ids, tgt, state=st, noise_fn=noise_fn, noise_state=state)
    torch.cuda.synchronize()
    full_s = (time.perf_counter() - t0) / full_steps
    clipped_frac = int(aux.num_clipped.sum().item()) / BLK_B
    print(f"[bench] full step {1e3 * full_s:.2f} ms, clipped fraction {clipped_frac:.3f}",
          file=sys.stderr, flush=True)

    # The clip -> sum -> noise part alone, on one step's captured operands.
    caps, _ = ghost_capture(model, per_example_lm_loss, ids, tgt)

    def step(st_, record):
        return ghost_clip_captured(caps, clipping_norm=C, noise_fn=noise_fn, noise_state=st_,
                                   gemm_events=record)

    for _ in range(max(1, args.warmup // 8)):
        _, state = step(state, None)
    steps = max(1, args.steps // 8)
    events = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        _, state = step(state, events)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    print(f"[bench] {steps} timed clip steps in {elapsed:.4f} s", file=sys.stderr, flush=True)
    gemm_ms = sum(a.elapsed_time(b) for a, b in events) / steps
    gram_f, gemm_f = block_flops()
    ms_per_step = 1e3 * elapsed / steps
    step_tflops = (gram_f + gemm_f) / (ms_per_step * 1e-3) / 1e12
    gemm_tflops = gemm_f / (gemm_ms * 1e-3) / 1e12
    cpu = None
    if not args.no_cpu_baseline:
        threads = cpu_threads()
        print(f"[bench] cpu baseline: 1 example on {threads} threads", file=sys.stderr, flush=True)
        cpu = {
            "value": block_cpu_baseline(threads),
            "unit": "examples/s",
            "cores": threads,
            "kind": "port",
            "sample": ("config 3 at B=1 (float32): the example's per-parameter gradients by its "
                       "own forward and backward (67.1M block parameters), streaming "
                       f"clip-and-sum, CPU randn noise; median of {CPU_REPEATS} steps after 1 warm-up; "
                       f"{cpu_host()}"),
        }
    return {
        "steps": steps,
        "warmup": max(1, args.warmup // 8),
        "ms_per_step": ms_per_step,
        "value": BLK_B * steps / elapsed,
        "config": {
            "workload": "Llama-style block d=2048, 16 heads, SwiGLU 8192, RMSNorm, RoPE, bf16, "
                        "B=16, T=1024, vocab 32000 (embedding and head frozen); ghost clipping "
                        "of the 67.1M block parameters from captured operands + fused "
                        "device-stream noise (BASELINE configs[2])",
            "global_batch": BLK_B,
            "seq_len": BLK_T,
            "clipping_norm": C,
            "noise_multiplier": NM,
            "normalize_by": 1.0,
            "clipped_fraction": clipped_frac,
            "step_tflops": step_tflops,
            "step_frac_of_bf16_peak": step_tflops / MFMA_BF16_PEAK_TFLOPS,
            "full_step_ms": 1e3 * full_s,
            "full_step_examples_per_s": BLK_B / full_s,
            "full_step": "forward + backward to the module outputs (PyTorch-ROCm, attention core "
                         "in float32) + ghost clip + sum + noise",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "clipped_sum_bf16_kernel<false, false> (dpc_clipped_sum_multi: the 4 "
                      "linear layers' 1024 output tiles in one launch per step)",
            "achieved": gemm_tflops,
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": gemm_tflops / MFMA_BF16_PEAK_TFLOPS,
            "avg_launch_ms": gemm_ms / max(1, len(events) // steps),
            "traffic": None,
        },
        "cpu_baseline": cpu,
    }


MLP_B = 256


def _mlp_ce(out, target):
    import torch

    return torch.nn.functional.cross_entropy(out, target, reduction="none")


def make_mlp():
    """The config-1 model, 784-512-10 with ReLU (torch's default Linear init)."""
    import torch

    class MLP(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.fc1 = torch.nn.Linear(784, 512)
            self.fc2 = torch.nn.Linear(512, 10)

        def forward(self, x):
            return self.fc2(torch.relu(self.fc1(x)))

    return MLP()


def mlp_cpu_baseline(threads: int, repeats: int = CPU_REPEATS):
    """The config-1 step as the reference runs it on the CPU: vmap(grad) of the
    per-example cross-entropy, the streaming clip-and-sum and the CPU-generator
    noise, at the full batch of 256.  Examples/s (median of ``repeats``)."""
    import torch

    from oracle import clip_oracle, ghost_oracle, noise_oracle

    torch.set_num_threads(threads)
    torch.manual_seed(0)
    model = make_mlp()
    params = {k: v.detach() for k, v in model.named_parameters()}
    g = torch.Generator().manual_seed(1)
    x = torch.randn(MLP_B, 784, generator=g)
    y = torch.randint(0, 10, (MLP_B,), generator=g)

    def step():
        per = ghost_oracle.mlp_per_example_grads(model, params, x, y)
        names = sorted(per)
        res = clip_oracle.stream_clip_and_sum([per[n] for n in names],
                                              clip_oracle.conservative_bound(C))
        draws = noise_oracle.draws_for(res.reduced, noise_oracle.step_seed(0, 0))
        return [noise_oracle.sample(v, NM * C, z) for v, z in zip(res.reduced, draws)]

    return median_rate(step, MLP_B, repeats)


def run_mlp(args) -> dict:
    import torch

    from opake_amd import _native
    from opake_amd.clipping import (
        GraphedGhostClip,
        ghost_capture,
        ghost_clip_captured,
        ghost_clipped_grad,
    )
    from opake_amd.noise import gaussian_noise
    from opake_amd.random import key

    _native.load()
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = make_mlp().to(dev)
    g = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn(MLP_B, 784, generator=g, device=dev)
    y = torch.randint(0, 10, (MLP_B,), generator=g, device=dev)
    noise_fn, state = gaussian_noise(noise_multiplier=NM, key=key(0), stream="device")
    fn, st = ghost_clipped_grad(model, _mlp_ce, clipping_norm=C)
    graphed = GraphedGhostClip(clipping_norm=C)

    def timed(step, n, warm):
        for _ in range(warm):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n

    holder = {"state": state}

    def full_eager():
        _, _, holder["state"] = fn(x, y, state=st, noise_fn=noise_fn, noise_state=holder["state"])

    def full_graphed():
        caps, _ = ghost_capture(model, _mlp_ce, x, y)
        _, holder["state"] = noise_fn(graphed(caps), holder["state"])

    caps, _ = ghost_capture(model, _mlp_ce, x, y)
    clip_eager_s = timed(lambda: ghost_clip_captured(caps, clipping_norm=C), args.steps,
                         args.warmup)
    clip_graph_s = timed(lambda: graphed(caps), args.steps, args.warmup)
    eager_s = timed(full_eager, args.steps, args.warmup)
    graph_s = timed(full_graphed, args.steps, args.warmup)
    print(f"[bench] clip eager {1e3 * clip_eager_s:.3f} ms, graphed {1e3 * clip_graph_s:.3f} ms; "
          f"full step eager {1e3 * eager_s:.3f} ms, graphed {1e3 * graph_s:.3f} ms",
          file=sys.stderr, flush=True)
    best = min(eager_s, graph_s)
    flops = 2 * MLP_B * (784 * 512 + 512 * 10)  # clipped sums (flat layers)
    cpu = None
    if not args.no_cpu_baseline:
        threads = cpu_threads()
        cpu = {
            "value": mlp_cpu_baseline(threads),
            "unit": "examples/s",
            "cores": threads,
            "kind": "port",
            "sample": ("config 1 in full (B=256, float32): vmap(grad) of the per-example "
                       "cross-entropy, streaming clip-and-sum, CPU randn noise; median of "
                       f"{CPU_REPEATS} steps after 1 warm-up; {cpu_host()}"),
        }
    return {
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": 1e3 * best,
        "value": MLP_B / best,
        "dtype": "fp32",
        "config": {
            "workload": "MLP 784-512-10 (ReLU), fp32, B=256 flat inputs, per-example "
                        "cross-entropy; full DP step on the GPU: forward, backward to the layer "
                        "outputs, ghost clip + sum (flat norms) and device-stream noise "
                        "(BASELINE configs[0])",
            "global_batch": MLP_B,
            "clipping_norm": C,
            "noise_multiplier": NM,
            "normalize_by": 1.0,
            "full_step_eager_ms": 1e3 * eager_s,
            "full_step_graphed_ms": 1e3 * graph_s,
            "clip_eager_ms": 1e3 * clip_eager_s,
            "clip_graphed_ms": 1e3 * clip_graph_s,
            "value_from": "graphed" if graph_s <= eager_s else "eager",
        },
        "roofline": {
            "bound": "latency",
            "kernel": "whole step (launch-bound at this size)",
            "achieved": flops / (clip_graph_s * 1e12),
            "peak": 157.3,
            "unit": "TFLOP/s",
            "frac": flops / (clip_graph_s * 1e12) / 157.3,
            "traffic": None,
        },
        "cpu_baseline": cpu,
    }


LORA_B, LORA_T, LORA_D, LORA_H, LORA_KV, LORA_F, LORA_R = 8, 2048, 4096, 32, 8, 14336, 16


def lora_model(device, dtype, seed=0):
    import torch

    from opake_amd.lora import LoRABlock

    torch.manual_seed(seed)
    model = LoRABlock(LORA_D, LORA_H, LORA_KV, LORA_F, LORA_R, 32.0, dtype=dtype, device=device)
    with torch.no_grad():
        for n, p in model.named_parameters():
            if ".lora_A." not in n:  # base weights, norms and lora_B: N(0, 0.02)
                p.normal_(0.0, 0.02) if p.dim() > 1 else p.fill_(1.0)
    return model


def lora_work(b=LORA_B, t=LORA_T):
    """Per-example adapter gradients: FLOPs (2 T din r per adapter side) and the
    algorithmic HBM bytes of their kernel -- every operand read once (q / k / v
    share their input, and so do gate / up: 3 of the 7 lora_A inputs are
    repeats) and the [B, dout, din] gradients written in bf16 -- summed over
    the 14 adapters."""
    kv = LORA_D // LORA_H * LORA_KV
    projs = [(LORA_D, LORA_D), (LORA_D, kv), (LORA_D, kv), (LORA_D, LORA_D),
             (LORA_D, LORA_F), (LORA_D, LORA_F), (LORA_F, LORA_D)]
    flops = nbytes = 0
    for din, dout in projs:
        for a, g in ((din, LORA_R), (LORA_R, dout)):
            flops += b * 2 * t * a * g
            nbytes += b * (t * (a + g) * 2 + a * g * 2)
    nbytes -= 3 * b * t * LORA_D * 2
    return flops, nbytes


def _mse_loss(out, target):
    return ((out.float() - target.float()) ** 2).mean(dim=(1, 2))


def lora_cpu_baseline(threads: int):
    """One example of the config-4 step on the CPU: the adapters' per-example
    gradients by the example's own forward and backward, the streaming
    clip-and-sum and the CPU-generator noise.  Examples/s."""
    import torch

    from oracle import clip_oracle, ghost_oracle, noise_oracle

    torch.set_num_threads(threads)
    model = lora_model(torch.device("cpu"), torch.float32, seed=1)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(1, LORA_T, LORA_D, generator=g)
    tgt = torch.randn(1, LORA_T, LORA_D, generator=g)

    def step():
        per = ghost_oracle.per_example_grads_loop(model, _mse_loss, (x,), tgt)
        names = sorted(per)
        res = clip_oracle.stream_clip_and_sum([per[n] for n in names],
                                              clip_oracle.conservative_bound(C))
        draws = noise_oracle.draws_for(res.reduced, noise_oracle.step_seed(0, 0))
        return [noise_oracle.sample(v, NM * C, z) for v, z in zip(res.reduced, draws)]

    return median_rate(step, 1)


def run_lora(args) -> dict:
    import torch

    from opake_amd import _native
    from opake_amd.clipping import ghost_capture, ghost_clip_captured, ghost_clipped_grad
    from opake_amd.noise import gaussian_noise
    from opake_amd.random import key

    _native.load()
    dev = torch.device("cuda:0")
    model = lora_model(dev, torch.bfloat16)
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(LORA_B, LORA_T, LORA_D, generator=g, device=dev).to(torch.bfloat16)
    tgt = torch.randn(LORA_B, LORA_T, LORA_D, generator=g, device=dev)
    noise_fn, state = gaussian_noise(noise_multiplier=NM, key=key(0), stream="device")

    fn, st = ghost_clipped_grad(model, _mse_loss, clipping_norm=C, return_aux=True)
    full_steps = max(1, args.steps // 20)
    for _ in range(max(1, args.warmup // 40)):
        (_, aux), _, state = fn(x, tgt, state=st, noise_fn=noise_fn, noise_state=state)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(full_steps):
        (_, aux), _, state = fn(x, tgt, state=st, noise_fn=noise_fn, noise_state=state)
    torch.cuda.synchronize()
    full_s = (time.perf_counter() - t0) / full_steps
    clipped_frac = int(aux.num_clipped.sum().item()) / LORA_B
    print(f"[bench] full step {1e3 * full_s:.2f} ms, clipped fraction {clipped_frac:.3f}",
          file=sys.stderr, flush=True)

    caps, _ = ghost_capture(model, _mse_loss, x, tgt)

    def step(st_, record):
        return ghost_clip_captured(caps, clipping_norm=C, noise_fn=noise_fn, noise_state=st_,
                                   gemm_events=record)

    for _ in range(max(1, args.warmup // 4)):
        _, state = step(state, None)
    steps = max(1, args.steps // 4)
    events = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        _, state = step(state, events)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    print(f"[bench] {steps} timed clip steps in {elapsed:.4f} s", file=sys.stderr, flush=True)
    kern_ms = sum(a.elapsed_time(b) for a, b in events) / steps
    flops, nbytes = lora_work()
    ms_per_step = 1e3 * elapsed / steps
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        threads = cpu_threads()
        print(f"[bench] cpu baseline: 1 example on {threads} threads", file=sys.stderr, flush=True)
        cpu = {
            "value": lora_cpu_baseline(threads),
            "unit": "examples/s",
            "cores": threads,
            "kind": "port",
            "sample": ("config 4 at B=1 (float32): the 14 adapters' gradients by the example's "
                       "own forward and backward, streaming clip-and-sum, CPU randn noise; "
                       f"median of {CPU_REPEATS} steps after 1 warm-up; {cpu_host()}"),
        }
    return {
        "steps": steps,
        "warmup": max(1, args.warmup // 4),
        "ms_per_step": ms_per_step,
        "value": LORA_B * steps / elapsed,
        "config": {
            "workload": "LoRA r=16 (alpha 32) on q/k/v/o/gate/up/down of an 8B-shaped block "
                        "(d=4096, FFN 14336, 32 heads / 8 KV heads), bf16, B=8, T=2048, base "
                        "frozen N(0,0.02), lora_A Kaiming-uniform, lora_B N(0,0.02); clipping "
                        "of the 1,310,720 adapter parameters from captured operands (direct "
                        "per-example gradients) + fused device-stream noise (BASELINE "
                        "configs[3])",
            "global_batch": LORA_B,
            "seq_len": LORA_T,
            "clipping_norm": C,
            "noise_multiplier": NM,
            "normalize_by": 1.0,
            "clipped_fraction": clipped_frac,
            "loss": "mean squared error to a N(0,1) target",
            "direct_tflops": flops / (kern_ms * 1e-3) / 1e12,
            "full_step_ms": 1e3 * full_s,
            "full_step_examples_per_s": LORA_B / full_s,
            "full_step": "forward + backward to the adapter outputs (PyTorch-ROCm, attention "
                         "core in float32) + clip + sum + noise",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "narrow_wide_mfma_kernel<16, 3> (dpc_per_example_grads_grouped: the 14 "
                      "adapter gradients in one launch per step, as 11 groups -- q / k / v and "
                      "gate / up each share one pass over their input)",
            "achieved": gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": gbs / HBM_PEAK_GBS,
            "avg_launch_ms": kern_ms,
            "traffic": None,
        },
        "cpu_baseline": cpu,
    }


def run_leaves(args) -> dict:
    """The materialised-leaf path (the reference's own streaming clip-and-sum,
    ``_streaming.py:39-185``, as ``dpc_leaves_*``) on the config-2 layer's
    per-example gradients, each HBM pass timed on its own: the norm pass, the
    clip factors, the scale-store-sum pass and the device-stream noise pass."""
    import math

    import torch

    from opake_amd import _native as nat
    from opake_amd import ops
    from opake_amd.clipping import _numerics as num
    from opake_amd.clipping._leaves import LeafBatch

    nat.load()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    # Per-example gradients [B, dout, din] in bf16, each example scaled so
    # that its norm is C * lognormal(0, 1): about half are clipped.
    P = DOUT * DIN
    z = torch.randn(B, 1, 1, generator=g, device=dev)
    leaf = (torch.randn(B, DOUT, DIN, generator=g, device=dev) * (C / math.sqrt(P)) *
            torch.exp(z)).to(torch.bfloat16)
    batch = LeafBatch([leaf])
    roundoff = num.norm_roundoff(torch.float32, torch.float64, 1, num.reduction_terms([P]))
    guards = [num.guard_constants(torch.bfloat16, torch.float32, roundoff)]
    stream = nat.stream_handle(dev)
    sq = torch.empty(B, dtype=torch.float64, device=dev)
    seed = 12345

    def step(ev):
        ev[0].record()
        leaf_sq = batch.sqnorms()
        ev[1].record()
        nat.call("dpc_row_sum_f64", nat.ptr(leaf_sq), B, 1, 0, nat.ptr(sq), stream)
        cf = ops.clip_factors(sq, num.conservative_bound(C), guards,
                              count_threshold=num.float32_of(C))
        ev[2].record()
        (center,), _ = batch.apply({torch.bfloat16: cf.scale[0:1]})
        ev[3].record()
        out = ops.add_noise(center, NM * C, mode=nat.NOISE_PHILOX, seed=seed, leaf_id=0)
        ev[4].record()
        return out, cf

    def events():
        return [torch.cuda.Event(enable_timing=True) for _ in range(5)]

    for _ in range(args.warmup):
        _, cf = step(events())
    torch.cuda.synchronize()
    clipped_frac = int(cf.nclipped.item()) / B
    evs = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        evs.append(events())
        step(evs[-1])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = [sum(e[i].elapsed_time(e[i + 1]) for e in evs) / len(evs) for i in range(4)]
    nbytes = [B * P * 2 + B * (P // 2048) * 8,  # norm: read the leaves, fp64 tile partials
              B * 8 + B * 8,                     # clip: tiny
              B * P * 2 + P * 2,                 # apply: read the leaves, write the bf16 sum
              P * 2 + P * 2]                     # noise: read and write the bf16 sum
    names = ["norm pass (dpc_leaves_sqnorm)", "clip factors (dpc_row_sum_f64 + dpc_clip_factors)",
             "scale-store-sum pass (dpc_leaves_apply)", "noise pass (dpc_add_noise, Philox)"]
    passes = []
    for name, t, nb in zip(names, ms, nbytes):
        gbs = nb / (t * 1e-3) / 1e9
        passes.append({"pass": name, "ms": t, "bytes": nb, "GB_per_s": gbs,
                       "frac_of_hbm_peak": gbs / HBM_PEAK_GBS})
    ms_per_step = 1e3 * elapsed / args.steps
    dom = max(range(4), key=lambda i: ms[i])
    return {
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "value": B * args.steps / elapsed,
        "config": {
            "workload": "materialised-leaf clip + sum + device-stream noise of the config-2 "
                        "layer's per-example gradients [32, 4096, 4096] bf16 (the reference's "
                        "streaming clip-and-sum, as the fused-backend seam runs it; the "
                        "gradients are synthetic, resident in HBM)",
            "global_batch": B,
            "clipping_norm": C,
            "noise_multiplier": NM,
            "clipped_fraction": clipped_frac,
            "passes": passes,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": names[dom],
            "achieved": passes[dom]["GB_per_s"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": passes[dom]["frac_of_hbm_peak"],
            "avg_launch_ms": ms[dom],
            "traffic": None,
        },
        "cpu_baseline": None,
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", type=int, choices=(1, 2, 3, 4, 5), default=2,
                    help="BASELINE configuration: 2 (default line), 1 (MLP), 3 (transformer "
                         "block), 4 (LoRA) or 5 (MoE)")
    ap.add_argument("--path", choices=("ghost", "leaves"), default="ghost",
                    help="config 2 only: the ghost-norm step (default line) or the materialised-"
                         "leaf passes over the layer's per-example gradients, each pass timed")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200,
                    help="untimed steps; ~0.15 s of work lets the GPU clocks settle")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample", type=int, default=8, help="examples in the CPU sample")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 device-to-device copies of MIB MiB (a plain copy kernel of "
                         "known size, for scaling the FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the step shards by examples with one all-reduce; not built here).",
              file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2

    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.randn(n, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n * 4, "copies": 5}), flush=True)
        return 0

    if args.config in (1, 3, 4, 5) or args.path == "leaves":
        runner = run_leaves if args.path == "leaves" else \
            {1: run_mlp, 3: run_block, 4: run_lora, 5: run_moe}[args.config]
        out = runner(args)
        line = {"metric": METRIC, "value": out["value"], "unit": "examples/s", "n_gpus": 1,
                "steps": out["steps"], "warmup": out["warmup"], "ms_per_step": out["ms_per_step"],
                "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                "dtype": out.get("dtype", "bf16"),
                "data": "synthetic", "config": out["config"],
                "roofline": add_sustained(out["roofline"], torch.device("cuda:0")),
                "cpu_baseline": out["cpu_baseline"]}
        print(json.dumps(line), flush=True)
        return 0

    from opake_amd import _native
    from opake_amd.clipping import ghost_clip_sum
    from opake_amd.noise import gaussian_noise
    from opake_amd.random import key

    _native.load()
    dev = torch.device("cuda:0")
    A, G = make_inputs(dev)
    noise_fn, state = gaussian_noise(noise_multiplier=NM, key=key(0), stream="device")

    gemm_events = []

    def step(st, record):
        (res, aux), st = ghost_clip_sum(A, G, clipping_norm=C, return_aux=True, noise_fn=noise_fn,
                                        noise_state=st, gemm_events=record)
        return res, aux, st

    # Clock settling (untimed, before the warm-up steps): the same step for
    # CLOCK_SETTLE_S of wall time, its results and noise state discarded.  A
    # process that starts on an idle GPU runs its first ~20 steps at a
    # quarter of the speed while the clocks come up (2.3 vs 0.53 ms per step
    # in a run timed after 5 warm-up steps); the settled rate is what a
    # training loop sees.  The W warm-up steps and the K timed steps follow
    # as requested.
    t_settle = time.perf_counter()
    n_settle = 0
    while time.perf_counter() - t_settle < CLOCK_SETTLE_S:
        step(state, None)
        n_settle += 1
        if n_settle % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        _, aux, state = step(state, None)
    torch.cuda.synchronize()
    clipped_frac = int(aux.num_clipped.item()) / B
    print(f"[bench] clock settling: {n_settle} untimed steps in {CLOCK_SETTLE_S} s; warmup done, "
          f"clipped fraction {clipped_frac:.3f}", file=sys.stderr, flush=True)

    torch.cuda.synchronize()
    # Timing events without the system-scope fence (dpc_timing_event_*):
    # torch's events cost this line 5-9 us per step and inflate the GEMM's
    # measured duration with the cache writeback and invalidation they do.
    pairs = [(_native.TimingEvent(), _native.TimingEvent()) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for pair in pairs:
        gemm_events.append(pair)
        _, aux, state = step(state, pair)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    print(f"[bench] {args.steps} timed steps in {elapsed:.4f} s", file=sys.stderr, flush=True)

    # Context measurements, after the timed steps (not part of the step):
    # the sustained MFMA rate (back-to-back MFMAs at full power for ~40 ms)
    # and the library reference of the same GEMM.
    sustained = sustained_mfma_tflops(dev)
    lib_ref = library_reference(A, G)
    print(f"[bench] context done: sustained {sustained:.0f} TFLOP/s, library GEMM "
          f"{lib_ref['natural_layout_ms']:.3f} ms", file=sys.stderr, flush=True)

    gemm_ms = sum(a.elapsed_time(b) for a, b in gemm_events) / len(gemm_events)
    gram_f, gemm_f = algorithmic_flops()
    total_f = gram_f + gemm_f
    ms_per_step = 1e3 * elapsed / args.steps
    examples_per_s = B * args.steps / elapsed
    step_tflops = total_f / (ms_per_step * 1e-3) / 1e12
    gemm_tflops = gemm_f / (gemm_ms * 1e-3) / 1e12

    cpu = None
    if not args.no_cpu_baseline:
        threads = cpu_threads()
        print(f"[bench] cpu baseline: {args.cpu_sample} examples on {threads} threads",
              file=sys.stderr, flush=True)
        rate = cpu_baseline(args.cpu_sample, threads)
        cpu = {
            "value": rate,
            "unit": "examples/s",
            "cores": threads,
            "kind": "port",
            "sample": (f"config 2 layer (4096x4096, T=512, bf16) at B={args.cpu_sample}: "
                       "vmap(grad) of the linear surrogate loss + streaming clip-and-sum + "
                       f"CPU randn noise; median of {CPU_REPEATS} steps after 1 warm-up; {cpu_host()}"),
        }

    line = {
        "metric": METRIC,
        "value": examples_per_s,
        "unit": "examples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": n_settle + args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "linear 4096x4096, B=32, T=512, bf16; ghost-norm clip + sum + fused "
                        "device-stream noise (BASELINE configs[1])",
            "untimed_steps": f"{n_settle + args.warmup}: {n_settle} clock-settling steps "
                             f"({CLOCK_SETTLE_S} s of wall time) then the {args.warmup} "
                             "requested warm-up steps",
            "global_batch": B,
            "seq_len": T,
            "clipping_norm": C,
            "noise_multiplier": NM,
            "normalize_by": 1.0,
            "G_scale": "N(0, C/sqrt(T*din*dout)) x lognormal(0,1) per example",
            "clipped_fraction": clipped_frac,
            "step_tflops": step_tflops,
            "step_frac_of_bf16_peak": step_tflops / MFMA_BF16_PEAK_TFLOPS,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "clipped_sum_bf16_kernel",
            "achieved": gemm_tflops,
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": gemm_tflops / MFMA_BF16_PEAK_TFLOPS,
            "avg_launch_ms": gemm_ms,
            "traffic": measured_traffic("clipped_sum_bf16_kernel"),
            "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1, "
                            "copy-calibrated; profiles/clipped_sum_cfg2_traffic.md)",
            "library_reference": lib_ref,
        },
        "cpu_baseline": cpu,
        "preparation": "sustained-MFMA measurement and library reference GEMM run after the "
                       "timed steps",
    }
    add_sustained(line["roofline"], dev, sustained)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
