"""Per-example clip -> sum (-> noise) of linear layers without per-example gradients.

The reference materialises every per-example gradient with ``vmap(grad)`` and
then runs the streaming clip-and-sum over them
(packages/opake-engine/src/opake/api/engine/clipping/_clipped_fun.py:676-695,
_streaming.py:39-185).  For a linear layer with inputs ``A`` [B, T, din] and
output gradients ``G`` [B, T, dout] the per-example weight gradient is
``G_i^T A_i``; this module computes the same clipped sum from ``A`` and ``G``:

1. per-example squared norms through the Gram identity
   ``||G_i^T A_i||^2 = <A_i A_i^T, G_i G_i^T>`` (``dpc_gram_sqnorms``; flat
   inputs use ``||a_i||^2 ||g_i||^2``), each with an upper bound ``err_i`` of
   its rounding error (the Gram inner product cancels, so its error scales
   with the Gram entries, not with the result);
2. guarded clip factors, the reference's ``_finalize_scale`` in float64
   (``dpc_clip_factors``) with the guard constants the reference would use for
   the materialised leaves (storage = leaf dtype, multiply = float32,
   roundoff from the leaf sizes), taken from ``sqrt(sq_i + err_i)``, so that
   ``c_i ||G_i^T A_i|| <= C`` holds exactly;
3. one GEMM ``sum_i c_i G_i^T A_i`` with ``/ normalize_by`` and, optionally,
   the Gaussian noise fused into its epilogue (``dpc_clipped_sum``).

Outputs use the reference's types: a ``ClippedPytree`` (or ``NoisedPytree``)
over ``{"weight": [dout, din]}`` (plus ``"bias": [dout]``) with
``max_norm = C / normalize_by``.

Differences from the materialised reference, all documented in tests:
* the norm is that of the exact product ``G_i^T A_i`` of the given values,
  not of its bf16-rounded copy (they agree to the bf16 rounding of the
  entries); the reported norms are the estimate ``sqrt(sq_i)``, the scales
  come from the bound (a clipped example is scaled by up to ~0.5% less at
  the bf16 benchmark shapes);
* the clipped sum never rounds an operand: on the bf16 MFMA path the
  products of the given values are summed in fp32 and each example's scale
  multiplies the fp32 accumulators (examples with extreme scales: G times the
  power of two of the scale, which is exact, and the mantissa on the
  accumulators); the reference instead rounds each ``c_i (G_i^T A_i)`` entry
  to the leaf dtype before its fp32 batch sum;
* an example whose ``A_i`` or ``G_i`` holds NaN/Inf is clipped the
  reference's way (its non-finite gradient entries zeroed, see
  ``_nonfinite``), with ``nonfinite="sanitize"`` (the default) outside HIP
  graph capture; with ``nonfinite="drop"`` (and under capture) it gets clip
  factor 0 and is left out.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch.autograd.profiler import record_function

from opake_amd import _native as nat
from opake_amd import ops
from opake_amd.clipping import _nonfinite as _nf
from opake_amd.clipping import _numerics as num
from opake_amd.clipping._leaves import _sum_dtype_of, leaves_clip_sum
from opake_amd.exceptions import ConfigurationError, InputTypeError
from opake_amd.noise import GaussianNoiseState, step_key_for
from opake_amd.random import generator_from_key
from opake_amd.types import ClippedPytree, NoisedPytree, PerGroup, clipped

_DEFAULT_GAMMA = 0.01


@dataclass(frozen=True)
class GhostClipAux:
    """Per-example diagnostics (device tensors; nothing is synchronised).

    ``grad_norms``: per-example gradient norms before clipping (float32, the
    reference's accumulation dtype).  ``clip_scales``: the guarded factors that
    were applied.  ``num_clipped``: int32 [1], examples with norm > C.
    ``clipped_grad_norms``: per-example norms after clipping, ``scale_i *
    norm_i`` (float32, computed on access; the clipped gradient is never
    formed).
    """

    grad_norms: torch.Tensor
    clip_scales: torch.Tensor
    num_clipped: torch.Tensor
    batch_size: int

    @property
    def clipped_grad_norms(self) -> torch.Tensor:
        return self.clip_scales * self.grad_norms

    @property
    def clipping_rate(self) -> float:
        """Fraction of clipped examples (synchronises the host)."""
        if self.batch_size == 0:
            return 0.0
        return float(self.num_clipped.item()) / float(self.batch_size)


def _check_inputs(A, G, bias):
    if not isinstance(A, torch.Tensor) or not isinstance(G, torch.Tensor):
        raise InputTypeError("A and G must be tensors")
    if A.dim() == 2 and G.dim() == 2:
        A, G = A.unsqueeze(1), G.unsqueeze(1)
    if A.dim() != 3 or G.dim() != 3 or A.shape[:2] != G.shape[:2]:
        raise ConfigurationError(
            "expected A [B, T, din] and G [B, T, dout] (or [B, din] / [B, dout]), got "
            f"{tuple(A.shape)} and {tuple(G.shape)}"
        )
    if A.dtype != G.dtype or A.dtype not in (torch.float32, torch.bfloat16):
        raise ConfigurationError("A and G must share a dtype: float32 or bfloat16")
    return A, G


def guard_for_linear(dtype: torch.dtype, din: int, dout: int, bias: bool):
    """(rel, abs) guard of the materialised weight (+ bias) leaves."""
    acc = num.compute_dtype_for_reduction([dtype])
    sizes = [dout * din] + ([dout] if bias else [])
    roundoff = num.norm_roundoff(acc, torch.float64, len(sizes), num.reduction_terms(sizes))
    multiply = torch.promote_types(dtype, acc)
    return num.guard_constants(dtype, multiply, roundoff)


def ghost_sqnorms(A: torch.Tensor, G: torch.Tensor, *, bias: bool = False,
                  out: torch.Tensor | None = None, err: torch.Tensor | None = None,
                  return_error: bool = True):
    """Per-example squared gradient norms of one linear layer and the bounds of
    their rounding errors: ``(sq, err)``, float64 [B] each, with
    ``sq + err >= ||G_i^T A_i||^2``.  With ``out`` / ``err`` the layer's values
    are added to them.  ``return_error=False`` returns ``sq`` alone (and
    accumulates into ``out`` without a bound): such norms are not a sound
    basis for a clip factor."""
    A, G = _check_inputs(A, G, bias)
    if not return_error and err is not None:
        raise ConfigurationError("err was given together with return_error=False")
    if A.shape[1] == 1:
        return ops.flat_sqnorms(A[:, 0], G[:, 0], with_bias=bias, out=out, err=err,
                                return_error=return_error)
    return ops.gram_sqnorms(A, G, with_bias=bias, out=out, err=err, return_error=return_error)


def _scale_kind(auto_s_gamma):
    if auto_s_gamma is None:
        return nat.SCALE_FIXED, 0.0
    if auto_s_gamma <= 0:
        raise ConfigurationError(f"gamma must be positive, got {auto_s_gamma}")
    return nat.SCALE_AUTO_S, float(auto_s_gamma)


def ghost_clip_sum(
    A: torch.Tensor,
    G: torch.Tensor,
    *,
    clipping_norm: float,
    normalize_by: float = 1.0,
    bias: bool = False,
    auto_s_gamma: float | None = None,
    dtype: torch.dtype | None = None,
    return_aux: bool = False,
    noise_fn=None,
    noise_state: GaussianNoiseState | None = None,
    gemm_events=None,
    nonfinite: str = "sanitize",
):
    """Clipped (and optionally noised) sum of a linear layer's per-example gradients.

    Without ``noise_fn``: returns ``ClippedPytree`` (or ``(ClippedPytree, aux)``).
    With ``noise_fn``/``noise_state`` from :func:`opake_amd.noise.gaussian_noise`:
    the noise is added in the GEMM epilogue and the call returns
    ``(NoisedPytree, next_state)`` (or ``((NoisedPytree, aux), next_state)``),
    bit-identical to ``noise_fn(ghost_clip_sum(...), noise_state)``.
    ``auto_s_gamma`` selects AUTO-S scaling ``C / (||g|| + gamma)``.
    ``gemm_events``: optional ``(start, end)`` pair of events (``torch.cuda.Event``
    or the fence-free ``opake_amd._native.TimingEvent``)
    recorded on the current stream around the clipped-sum launch (timing hook).
    ``nonfinite``: ``"sanitize"`` clips an example whose operands hold NaN/Inf
    from its sanitised gradient, as the reference does (the host reads a
    count the norm pass leaves in pinned memory); ``"drop"`` leaves it out.
    """
    if isinstance(clipping_norm, PerGroup):
        raise ConfigurationError("per-group clipping is not supported by ghost_clip_sum")
    if clipping_norm <= 0:
        raise ConfigurationError(f"clipping_norm must be positive, got {clipping_norm}")
    if normalize_by <= 0.0:
        raise ConfigurationError(f"normalize_by must be > 0, got {normalize_by}.")
    A, G = _check_inputs(A, G, bias)
    B, T, din = A.shape
    dout = G.shape[2]
    out_dtype = dtype or A.dtype
    kind, gamma = _scale_kind(auto_s_gamma)
    max_norm = clipping_norm / normalize_by

    if noise_fn is not None and noise_fn.compute_dtype != torch.float32:
        # The GEMM epilogue adds noise in float32; another compute dtype adds
        # it after the clipped sum, through noise_fn itself.
        if noise_state is None:
            raise ConfigurationError("noise_state is required with noise_fn")
        out = ghost_clip_sum(A, G, clipping_norm=clipping_norm, normalize_by=normalize_by,
                             bias=bias, auto_s_gamma=auto_s_gamma, dtype=dtype,
                             return_aux=return_aux, gemm_events=gemm_events,
                             nonfinite=nonfinite)
        res, aux = out if return_aux else (out, None)
        res, next_state = noise_fn(res, noise_state)
        return ((res, aux) if return_aux else res), next_state

    watch = _nf.watch(A.device, 1, nonfinite)
    flag = watch.slot(0) if watch is not None else None
    with record_function("opake::ghost_clip_sum"):
        guards = [guard_for_linear(A.dtype, din, dout, bias)]
        bound = num.conservative_bound(clipping_norm)
        threshold = num.float32_of(clipping_norm)
        if T > 1:
            # Norms and clip factors in one launch where the split Gram kernel applies.
            sq, err, cf = ops.gram_clip_factors(A, G, bound, guards, with_bias=bias, kind=kind,
                                                gamma=gamma, count_threshold=threshold,
                                                nonfinite=flag)
        else:
            sq, err = ghost_sqnorms(A, G, bias=bias)
            cf = ops.clip_factors(sq, bound, guards, err=err, kind=kind, gamma=gamma,
                                  count_threshold=threshold, nonfinite=flag)
        spec = None
        next_state = None
        std = 0.0
        if noise_fn is not None:
            if noise_state is None:
                raise ConfigurationError("noise_state is required with noise_fn")
            std = noise_fn.clipped_stddev(clipped(None, max_norm=max_norm))
            if std != 0.0:
                step_key = step_key_for(noise_state)
                # Flatten order of {"bias", "weight"}: bias first when present.
                w_leaf, b_leaf = (1, 0) if bias else (0, 0)
                if noise_fn.stream == "reference":
                    gen = generator_from_key(step_key)
                    b_draw = torch.randn(dout, dtype=torch.float32, generator=gen) if bias else None
                    w_draw = torch.randn((dout, din), dtype=torch.float32, generator=gen)
                    dev = A.device
                    spec = ops.NoiseSpec(
                        sigma=std,
                        mode=nat.NOISE_INJECTED,
                        noise=w_draw.pin_memory().to(dev, non_blocking=True),
                        bias_noise=(b_draw.pin_memory().to(dev, non_blocking=True)
                                    if bias else None),
                    )
                else:
                    spec = ops.NoiseSpec(sigma=std, mode=nat.NOISE_PHILOX, seed=step_key.seed,
                                         leaf_id=w_leaf, bias_leaf_id=b_leaf)
            next_state = GaussianNoiseState(
                _step_counter=noise_state._step_counter + 1, _rng_key=noise_state._rng_key)
        if gemm_events is not None:
            gemm_events[0].record()
        w, b = ops.clipped_sum(
            A, G, cf.scale[0], plan=cf.plan[0], normalize_by=normalize_by, noise=spec,
            out_dtype=out_dtype, with_bias=bias,
        )
        if gemm_events is not None:
            gemm_events[1].record()
    tree = {"weight": w}
    if bias:
        tree["bias"] = b
    if watch is not None and watch.count() > 0:
        _clip_nonfinite_examples(A, G, sq, err, cf, tree, bias=bias, clipping_norm=clipping_norm,
                                 kind=kind, gamma=gamma, normalize_by=normalize_by,
                                 threshold=threshold)
    aux = GhostClipAux(grad_norms=cf.norms, clip_scales=cf.scale[0], num_clipped=cf.nclipped,
                       batch_size=B)
    if noise_fn is None:
        result = clipped(tree, max_norm=max_norm)
        return (result, aux) if return_aux else result
    result = NoisedPytree(pytree=tree, max_norm=max_norm, noise_stddev=std)
    return ((result, aux) if return_aux else result), next_state


def _clip_nonfinite_examples(A, G, sq, err, cf, tree, *, bias, clipping_norm, kind, gamma,
                             normalize_by, threshold):
    """The examples whose norm is not finite (their operands hold NaN/Inf),
    clipped from their sanitised per-example gradients by the leaf kernels and
    added to ``tree``; their norms, scales and the clipped count in ``cf``
    are replaced."""
    bad = _nf.bad_examples(sq, err)
    if bad.numel() == 0:
        return
    pdt = A.dtype
    w, b = _nf.sanitized_linear_grads(A[bad], G[bad], pdt, bias)
    leaves = [b, w] if bias else [w]  # flatten order: "bias" < "weight"
    out_dtype = tree["weight"].dtype
    res = leaves_clip_sum(leaves, float(clipping_norm),
                          kind="auto_s" if kind == nat.SCALE_AUTO_S else "fixed", gamma=gamma,
                          sum_dtypes={pdt: (_sum_dtype_of(pdt, None), out_dtype)})
    sums = res.reduced if bias else [None, res.reduced[0]]
    for name, x in zip(("bias", "weight"), sums):
        if x is None:
            continue
        if normalize_by != 1.0:
            x = x / normalize_by
        tree[name] = (tree[name] + x).to(out_dtype)
    cf.norms[bad] = res.norms
    cf.scale[0][bad] = res.scales[pdt][0]
    cf.nclipped.copy_((cf.norms > threshold).sum().reshape(1).to(torch.int32))


__all__ = ["GhostClipAux", "ghost_clip_sum", "ghost_sqnorms", "guard_for_linear"]
