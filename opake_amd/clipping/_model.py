"""Model-level ghost clipping: clip -> sum (-> noise) over every linear layer.

The reference differentiates ``loss_fn`` per example with ``vmap(grad)``
(packages/opake-engine/src/opake/api/engine/clipping/_clipped_grad.py:278-296)
and clips the materialised gradients (_streaming.py:39-185).  For a model whose
trainable parameters all sit in ``nn.Linear`` layers, the same clipped sum
follows from each layer's inputs ``A`` and output gradients ``G`` alone:

1. one ordinary batched forward of the model on PyTorch-ROCm, with forward
   hooks that keep every linear layer's input ``A`` and output, then
   ``autograd.grad(sum_i loss_i, outputs)`` for the output gradients ``G``
   (``G_i`` is example ``i``'s own output gradient because ``loss_i`` depends on
   example ``i`` only; no weight-gradient GEMM runs);
2. per-example squared norms summed over layers (``dpc_gram_sqnorms`` /
   ``dpc_flat_sqnorms``, accumulated into one float64 [B] vector);
3. one set of guarded clip factors for the whole parameter tree, with the
   reference's roundoff for the materialised leaves (``_norm_roundoff`` over
   all weights and biases);
4. one ``dpc_clipped_sum`` per layer (weight and bias), with ``/ normalize_by``
   and, optionally, the Gaussian noise fused into the epilogue.

The output is the reference's ``ClippedPytree`` (``NoisedPytree`` with noise)
over ``{parameter name: tensor}`` with ``max_norm = C / normalize_by``; noise
leaves are drawn in sorted-name (flatten) order.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch.autograd.profiler import record_function

from opake_amd import _native as nat
from opake_amd import ops
from opake_amd.clipping import _numerics as num
from opake_amd.clipping._clipped_fun import FixedClipState
from opake_amd.exceptions import ConfigurationError, InputTypeError
from opake_amd.noise import GaussianNoiseState, step_key_for
from opake_amd.random import generator_from_key
from opake_amd.types import NoisedPytree, PerGroup, clipped


@dataclass(frozen=True)
class GhostGradAux:
    """Per-example diagnostics (device tensors): loss values, norms before
    clipping (float32), applied clip scales, ``num_clipped`` (int32 [1])."""

    loss_values: torch.Tensor
    grad_norms: torch.Tensor
    clip_scales: torch.Tensor
    num_clipped: torch.Tensor
    batch_size: int

    @property
    def clipping_rate(self) -> float:
        if self.batch_size == 0:
            return 0.0
        return float(self.num_clipped.item()) / float(self.batch_size)


class _Capture:
    """Forward hook that keeps a linear layer's input and its (graph-attached) output."""

    def __init__(self, module: torch.nn.Linear):
        self.A = None
        self.out = None
        self._handle = module.register_forward_hook(self._fwd)

    def _fwd(self, module, inputs, output):
        self.A = inputs[0].detach()
        self.out = output

    def remove(self):
        self._handle.remove()


def _linear_layers(model: torch.nn.Module):
    layers = []
    covered = set()
    for name, mod in model.named_modules():
        if isinstance(mod, torch.nn.Linear) and mod.weight.requires_grad:
            layers.append((name, mod))
            covered.add(id(mod.weight))
            if mod.bias is not None:
                covered.add(id(mod.bias))
    for pname, p in model.named_parameters():
        if p.requires_grad and id(p) not in covered:
            raise ConfigurationError(
                f"parameter {pname!r} is trainable but not part of an nn.Linear layer; "
                "ghost clipping covers linear layers only (freeze it or use clipped_grad)")
    if not layers:
        raise ConfigurationError("the model has no trainable nn.Linear layer")
    return layers


def _as_btd(x: torch.Tensor, B: int) -> torch.Tensor:
    """[B, d] -> [B, 1, d]; [B, ..., d] -> [B, T, d] with T the product of the middle dims."""
    if x.shape[0] != B:
        raise ConfigurationError("a linear layer's input does not have the batch as dim 0")
    return x.reshape(B, -1, x.shape[-1])


def ghost_clipped_grad(
    model: torch.nn.Module,
    loss_fn,
    *,
    clipping_norm: float,
    normalize_by: float = 1.0,
    return_aux: bool = False,
    dtype: torch.dtype | None = None,
):
    """Create ``grad_fn(inputs, targets, *, state, noise_fn=None, noise_state=None)``.

    ``loss_fn(outputs, targets)`` must return per-example losses ``[B]``
    (e.g. ``cross_entropy(..., reduction="none")``).  Without ``noise_fn`` the
    call returns ``(ClippedPytree, state)``; with it, ``(NoisedPytree, state,
    noise_state')`` where the noise was fused into the clipped-sum epilogue.
    With ``return_aux`` the first element is ``(result, GhostGradAux)``.
    """
    if isinstance(clipping_norm, PerGroup):
        raise ConfigurationError("per-group clipping is not supported by ghost_clipped_grad")
    if isinstance(clipping_norm, bool) or not isinstance(clipping_norm, (int, float)):
        raise InputTypeError(f"clipping_norm must be a float, got {type(clipping_norm)}")
    if clipping_norm <= 0:
        raise ConfigurationError(f"clipping_norm must be positive, got {clipping_norm}")
    if normalize_by <= 0.0:
        raise ConfigurationError(f"normalize_by must be > 0, got {normalize_by}.")
    layers = _linear_layers(model)
    max_norm = clipping_norm / normalize_by
    state0 = FixedClipState()

    # Output leaves, in flatten (sorted-name) order.
    leaf_names = []
    for name, mod in layers:
        leaf_names.append(f"{name}.weight")
        if mod.bias is not None:
            leaf_names.append(f"{name}.bias")
    leaf_names.sort()
    leaf_index = {n: i for i, n in enumerate(leaf_names)}

    def grad_fn(inputs, targets, *, state, noise_fn=None, noise_state=None):
        captures = [_Capture(mod) for _, mod in layers]
        try:
            with record_function("opake::ghost_clipped_grad"), torch.enable_grad():
                outputs = model(inputs)
                losses = loss_fn(outputs, targets)
                if losses.dim() != 1:
                    raise ConfigurationError("loss_fn must return per-example losses [B]")
                B = losses.shape[0]
                for (name, _), cap in zip(layers, captures):
                    if cap.out is None:
                        raise ConfigurationError(f"layer {name!r} was not used by the forward pass")
                # Gradients with respect to the layer outputs only: autograd
                # prunes the weight-gradient GEMMs, which the clipped sum replaces.
                grads = torch.autograd.grad(losses.sum(), [c.out for c in captures],
                                            allow_unused=True)
        finally:
            for c in captures:
                c.remove()
        pairs = []
        for (name, mod), cap, g in zip(layers, captures, grads):
            A = _as_btd(cap.A, B)
            G = _as_btd(g.detach() if g is not None else torch.zeros_like(cap.out), B)
            if A.dtype != G.dtype:
                G = G.to(A.dtype)
            pairs.append((name, mod, A.contiguous(), G.contiguous()))
            cap.out = None

        sq = None
        for name, mod, A, G in pairs:
            bias = mod.bias is not None
            if A.shape[1] == 1:
                sq = ops.flat_sqnorms(A[:, 0], G[:, 0], with_bias=bias, out=sq)
            else:
                sq = ops.gram_sqnorms(A, G, with_bias=bias, out=sq)

        # Guards for the materialised leaves the reference would clip.
        sizes = []
        for _, mod, _, _ in pairs:
            sizes.append(mod.weight.numel())
            if mod.bias is not None:
                sizes.append(mod.bias.numel())
        roundoff = num.norm_roundoff(torch.float32, torch.float64, len(sizes),
                                     num.reduction_terms(sizes))
        storage = sorted({A.dtype for _, _, A, _ in pairs}, key=str)
        guards = [num.guard_constants(dt, torch.promote_types(dt, torch.float32), roundoff)
                  for dt in storage]
        cf = ops.clip_factors(sq, num.conservative_bound(clipping_norm), guards,
                              count_threshold=num.float32_of(clipping_norm))

        std = 0.0
        gen = None
        step_key = None
        next_noise_state = None
        if noise_fn is not None:
            if noise_state is None:
                raise ConfigurationError("noise_state is required with noise_fn")
            std = noise_fn.clipped_stddev(clipped(None, max_norm=max_norm))
            if std != 0.0 and noise_fn.compute_dtype != torch.float32:
                raise ConfigurationError("fused noise supports compute_dtype float32 only")
            step_key = step_key_for(noise_state)
            if std != 0.0 and noise_fn.stream == "reference":
                gen = generator_from_key(step_key)
            next_noise_state = GaussianNoiseState(
                _step_counter=noise_state._step_counter + 1, _rng_key=noise_state._rng_key)

        # Reference-stream draws, one generator, flatten order.
        draws = {}
        if gen is not None:
            shapes = {}
            for name, mod, _, _ in pairs:
                shapes[f"{name}.weight"] = tuple(mod.weight.shape)
                if mod.bias is not None:
                    shapes[f"{name}.bias"] = tuple(mod.bias.shape)
            for leaf in leaf_names:
                draws[leaf] = torch.randn(shapes[leaf], dtype=torch.float32, generator=gen)

        tree = {}
        for name, mod, A, G in pairs:
            si = storage.index(A.dtype)
            spec = None
            if std != 0.0:
                wn, bn = f"{name}.weight", f"{name}.bias"
                if gen is not None:
                    dev = A.device
                    spec = ops.NoiseSpec(
                        sigma=std, mode=nat.NOISE_INJECTED,
                        noise=draws[wn].pin_memory().to(dev, non_blocking=True),
                        bias_noise=(draws[bn].pin_memory().to(dev, non_blocking=True)
                                    if mod.bias is not None else None))
                else:
                    spec = ops.NoiseSpec(sigma=std, mode=nat.NOISE_PHILOX, seed=step_key.seed,
                                         leaf_id=leaf_index[wn],
                                         bias_leaf_id=leaf_index.get(bn, 0))
            w, b = ops.clipped_sum(A, G, cf.scale[si], plan=cf.plan if len(storage) == 1 else None,
                                   normalize_by=normalize_by, noise=spec,
                                   out_dtype=dtype or mod.weight.dtype,
                                   with_bias=mod.bias is not None)
            tree[f"{name}.weight"] = w
            if mod.bias is not None:
                tree[f"{name}.bias"] = b
        tree = {k: tree[k] for k in leaf_names}
        if noise_fn is None:
            result = clipped(tree, max_norm=max_norm)
        else:
            result = NoisedPytree(pytree=tree, max_norm=max_norm, noise_stddev=std)
        if return_aux:
            aux = GhostGradAux(loss_values=losses.detach(), grad_norms=cf.norms,
                               clip_scales=cf.scale, num_clipped=cf.nclipped, batch_size=B)
            result = (result, aux)
        if noise_fn is None:
            return result, state
        return result, state, next_noise_state

    return grad_fn, state0


__all__ = ["GhostGradAux", "ghost_clipped_grad"]
