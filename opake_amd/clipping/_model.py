"""Model-level ghost clipping: clip -> sum (-> noise) over a model's parameters.

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
   ``dpc_flat_sqnorms``), one float64 [B] row per clipping group;
3. guarded clip factors per group, with the reference's roundoff for the
   materialised leaves (``_norm_roundoff`` over all weights and biases);
4. one ``dpc_clipped_sum`` per layer (weight and bias), with ``/ normalize_by``
   and, optionally, the Gaussian noise fused into the epilogue.

Row-segmented layers.  A module that feeds one linear layer with the rows of
several examples -- the experts of a mixture-of-experts layer, whose input is
the tokens routed to that expert -- sets ``linear.dpc_row_segments`` to the
per-example row counts (a list of B ints, rows in example order) before it
calls the layer.  Such a layer's per-example gradient is the sum over its
segment (the reference's "virtual experts" ``b * E + e``,
packages/opake-patches/src/opake/api/patches/kernels/fused_moe.py:20-27), and
all segmented layers of one shape go through one grouped norm launch
(``dpc_grouped_gram_sqnorms``) and one grouped clipped-sum launch
(``dpc_grouped_clipped_sum``).

``clipping_norm`` may be a ``PerGroup`` over the output leaves (keys
``"<layer>.weight"`` / ``"<layer>.bias"``, the parameter names): each group is clipped to its own
bound by its own per-example norm (_streaming.py:63-104), and the noise of a
leaf uses its group's standard deviation.

Other modules that own trainable parameters (RMSNorm / LayerNorm weights,
...) get their per-example gradients materialised -- ``vmap`` over the batch
of the module's own ``vjp`` from its captured inputs and output gradients,
which for such parameters is a few values per example -- and clipped with the
rest by the leaf kernels.

The output is the reference's ``ClippedPytree`` (``NoisedPytree`` with noise)
over ``{parameter name: tensor}`` with ``max_norm = C / normalize_by``; noise
leaves are drawn in sorted-name (flatten) order.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, replace

import numpy as np
import torch
from torch.autograd.profiler import record_function

from opake_amd import _native as nat
from opake_amd import ops
from opake_amd._tables import device_table
from opake_amd.clipping import _nonfinite as _nf
from opake_amd.clipping import _numerics as num
from opake_amd.clipping._clipped_fun import FixedClipState
from opake_amd.clipping._leaves import LeafBatch, _sum_dtype_of, leaves_clip_sum
from opake_amd.exceptions import ConfigurationError, InputTypeError
from opake_amd.noise import GaussianNoiseState, step_key_for
from opake_amd.pytree import param_path
from opake_amd.random import generator_from_key
from opake_amd.types import NoisedPytree, PerGroup, clipped


@dataclass(frozen=True)
class GhostGradAux:
    """Per-example diagnostics (device tensors): loss values, norms before
    clipping (float32 [B]), applied clip scales (float32 [n_guards, B] per
    group), ``num_clipped`` (int32 [1], or [G] per group), and per-group norms
    ``{group: float32 [B]}`` with ``PerGroup`` clipping; ``clipped_grad_norms``
    from them."""

    loss_values: torch.Tensor | None
    grad_norms: torch.Tensor
    clip_scales: torch.Tensor
    num_clipped: torch.Tensor
    batch_size: int
    group_norms: dict | None = None

    @property
    def clipped_grad_norms(self) -> torch.Tensor:
        """Per-example norms after clipping (``ClippedGradAux.clipped_grad_norms``,
        _clipped_grad.py:34-61): ``scale_i * norm_i``, per group then combined
        (float32, computed on access; the clipped gradient is never formed)."""
        if self.group_norms is None:
            return self.clip_scales[0] * self.grad_norms
        parts = [self.clip_scales[k][0].double() * self.group_norms[n].double()
                 for k, n in enumerate(sorted(self.group_norms))]
        return torch.sqrt(sum(p * p for p in parts)).to(torch.float32)

    @property
    def clipping_rate(self) -> float | None:
        if self.group_norms is not None:
            return None
        if self.batch_size == 0:
            return 0.0
        return float(self.num_clipped.sum().item()) / float(self.batch_size)


class _Capture:
    """Forward hook that keeps a linear layer's input, its (graph-attached)
    output and the row segments the caller declared for this call."""

    def __init__(self, module: torch.nn.Linear):
        self.A = None
        self.out = None
        self.segments = None
        self.calls = 0
        self._handle = module.register_forward_hook(self._fwd)

    def _fwd(self, module, inputs, output):
        self.calls += 1
        self.A = inputs[0].detach()
        self.out = output
        seg = getattr(module, "dpc_row_segments", None)
        self.segments = None if seg is None else [int(v) for v in seg]

    def remove(self):
        self._handle.remove()


def _trainable_modules(model: torch.nn.Module):
    """Linear layers with a trainable weight, and the other modules that own
    trainable parameters directly (``[(name, module, [(param name, param)])]``)."""
    linears, others = [], []
    seen = set()
    for name, mod in model.named_modules():
        own = [(pn, p) for pn, p in mod.named_parameters(recurse=False) if p.requires_grad]
        if not own:
            continue
        for _, p in own:
            if id(p) in seen:
                raise ConfigurationError(
                    f"module {name!r} shares a trainable parameter with another module")
            seen.add(id(p))
        if isinstance(mod, torch.nn.Linear) and mod.weight.requires_grad:
            if mod.bias is not None and not mod.bias.requires_grad:
                raise ConfigurationError(
                    f"layer {name!r}: a frozen bias under a trainable weight is not supported")
            linears.append((name, mod))
        else:
            others.append((name, mod, own))
    if not linears and not others:
        raise ConfigurationError("the model has no trainable parameter")
    return linears, others


class _DirectHook:
    """Forward hook of a module with its own trainable parameters (not a
    linear layer): keeps its positional inputs and its output."""

    def __init__(self, module: torch.nn.Module):
        self.args = None
        self.out = None
        self.calls = 0
        self._handle = module.register_forward_hook(self._fwd)

    def _fwd(self, module, inputs, output):
        self.calls += 1
        self.args = tuple(x.detach() if isinstance(x, torch.Tensor) else x for x in inputs)
        self.out = output

    def remove(self):
        self._handle.remove()


def _per_example_param_grads(mod, own, args, G):
    """Per-example gradients of ``mod``'s own parameters from its inputs and
    output gradients: ``vmap`` over the batch of the module's ``vjp`` (the
    reference's per-example ``grad``, restricted to this module).  Returns
    ``{param name: [B, *shape]}`` in the parameters' dtype."""
    from torch.func import functional_call, vjp, vmap

    params = {pn: p.detach() for pn, p in own}
    tensor_pos = [i for i, a in enumerate(args) if isinstance(a, torch.Tensor)]

    def single(p, g, *xs):
        full = list(args)
        for i, x in zip(tensor_pos, xs):
            full[i] = x.unsqueeze(0)

        def f(pp):
            return functional_call(mod, pp, tuple(full))

        _, fn = vjp(f, p)
        return fn(g.unsqueeze(0))[0]

    xs = [args[i] for i in tensor_pos]
    return vmap(single, in_dims=(None, 0) + (0,) * len(xs))(params, G, *xs)


def _as_btd(x: torch.Tensor, B: int) -> torch.Tensor:
    """[B, d] -> [B, 1, d]; [B, ..., d] -> [B, T, d] with T the product of the middle dims."""
    if x.shape[0] != B:
        raise ConfigurationError("a linear layer's input does not have the batch as dim 0")
    return x.reshape(B, -1, x.shape[-1])


def _validate_bound(clipping_norm) -> None:
    if isinstance(clipping_norm, PerGroup):
        for gname, value in clipping_norm.values.items():
            if value <= 0:
                raise ConfigurationError(
                    f"clipping_norm must be positive for all groups, got {value} for group "
                    f"'{gname}'")
        return
    if isinstance(clipping_norm, bool) or not isinstance(clipping_norm, (int, float)):
        raise InputTypeError(f"clipping_norm must be a float, got {type(clipping_norm)}")
    if clipping_norm <= 0:
        raise ConfigurationError(f"clipping_norm must be positive, got {clipping_norm}")


@dataclass
class LinearCapture:
    """One linear layer's operands for ghost clipping.

    ``A`` / ``G``: the layer's inputs and output gradients, ``[B, T, d]`` or
    ``[B, d]`` -- or, with ``segments`` (B per-example row counts), ``[rows,
    d]`` rows of several examples in example order.  The output leaves are
    ``"<name>.weight"`` (``[dout, din]``) and, with ``has_bias``,
    ``"<name>.bias"``; ``param_dtype`` is their default dtype (the operand
    dtype when ``None``).
    """

    name: str
    A: torch.Tensor
    G: torch.Tensor
    has_bias: bool = False
    segments: list | None = None
    param_dtype: torch.dtype | None = None
    norm_method: str = "auto"


def _direct_is_cheaper(T: int, din: int, dout: int) -> bool:
    """Per-example gradients (2 T din dout FLOP, kept for a layer with a side of
    at most 32, e.g. a LoRA adapter) against the Gram norm (T^2 (din + dout))."""
    return min(din, dout) <= ops.NARROW_MAX and 2 * din * dout < T * (din + dout)


@dataclass
class DirectCapture:
    """Materialised per-example gradients of parameters outside linear layers
    (norm weights, biases of other modules, ...): ``{leaf name: [B, *shape]}``.
    They are clipped with the linear layers' leaves by the leaf kernels
    (``dpc_leaves_sqnorm`` / ``dpc_leaves_apply``), the reference's own path
    for materialised values (_streaming.py:39-185)."""

    grads: dict


@dataclass
class _Layer:
    cap: LinearCapture
    group: int
    A: torch.Tensor  # dense [B, T, din]; segmented [rows, din]
    G: torch.Tensor

    @property
    def name(self):
        return self.cap.name


def _groups_of(leaf_names, clipping_norm):
    """Leaf -> group index, group names (sorted) and bounds."""
    if not isinstance(clipping_norm, PerGroup):
        return dict.fromkeys(leaf_names, 0), None, [float(clipping_norm)]
    group_names = sorted(clipping_norm.values)
    keys = {param_path(n) for n in leaf_names}
    mapped = set(clipping_norm.groups)
    if keys != mapped:
        missing = sorted(map(str, keys - mapped))
        extra = sorted(map(str, mapped - keys))
        raise ConfigurationError(
            "PerGroup path keys must match the pytree tensor leaves exactly."
            + (f" Leaves with no group assignment: {missing}." if missing else "")
            + (f" Group paths with no matching leaf: {extra}." if extra else ""))
    gidx = {n: k for k, n in enumerate(group_names)}
    leaf_group = {n: gidx[clipping_norm.groups[param_path(n)]] for n in leaf_names}
    return leaf_group, group_names, [float(clipping_norm.values[n]) for n in group_names]


def _event_pair(sink):
    """Record a start event on the current stream (the one the kernels use)."""
    if sink is None:
        return None
    pair = (nat.TimingEvent(), nat.TimingEvent())
    pair[0].record()
    sink.append(pair)
    return pair


def _close_pair(pair):
    if pair is not None:
        pair[1].record()


def ghost_clip_captured(
    captures,
    *,
    clipping_norm,
    normalize_by: float = 1.0,
    noise_fn=None,
    noise_state=None,
    dtype: torch.dtype | None = None,
    return_aux: bool = False,
    gemm_events: list | None = None,
    auto_s_gamma: float | None = None,
    nonfinite: str = "sanitize",
):
    """Clip -> sum (-> noise) from the captured operands of linear layers.

    ``captures``: a list of :class:`LinearCapture` (one per layer, all with
    the same batch).  Returns what ``ghost_clipped_grad``'s step returns,
    without the forward: ``ClippedPytree`` (``(NoisedPytree, noise_state')``
    with ``noise_fn``), and with ``return_aux`` the first element is
    ``(result, GhostGradAux)`` whose ``loss_values`` is ``None``.
    ``gemm_events`` (timing hook): a list that receives one pair of recorded
    timing events (``TimingEvent``: fence-free, ``elapsed_time`` like
    ``torch.cuda.Event``) around each clipped-sum launch (and each per-example
    gradient launch of a layer that takes the direct method).
    ``auto_s_gamma``: AUTO-S scaling ``R / (||g|| + gamma)`` with ``R =
    clipping_norm`` (``_auto.py:211-367``) instead of ``min(1, C / ||g||)``.
    ``nonfinite``: ``"sanitize"`` (default) clips an example whose operands
    hold NaN/Inf from its sanitised per-example gradients, as the reference
    does; ``"drop"`` leaves it out (as happens under HIP-graph capture).
    """
    _validate_bound(clipping_norm)
    kind, gamma = _scale_kind(auto_s_gamma)
    if normalize_by <= 0.0:
        raise ConfigurationError(f"normalize_by must be > 0, got {normalize_by}.")
    if not captures:
        raise ConfigurationError("no layers to clip")
    if noise_fn is not None and noise_fn.compute_dtype != torch.float32:
        # The epilogues add noise in float32; another compute dtype adds it
        # after the clipped sums, through noise_fn itself.
        if noise_state is None:
            raise ConfigurationError("noise_state is required with noise_fn")
        out = ghost_clip_captured(captures, clipping_norm=clipping_norm,
                                  normalize_by=normalize_by, dtype=dtype,
                                  return_aux=return_aux, gemm_events=gemm_events,
                                  auto_s_gamma=auto_s_gamma, nonfinite=nonfinite)
        res, aux = out if return_aux else (out, None)
        res, next_state = noise_fn(res, noise_state)
        return ((res, aux) if return_aux else res), next_state
    max_norm = clipping_norm / normalize_by
    per_group = isinstance(clipping_norm, PerGroup)
    direct = {}
    for c in captures:
        if isinstance(c, DirectCapture):
            for n, t in c.grads.items():
                if n in direct:
                    raise ConfigurationError(f"leaf {n!r} is given twice")
                direct[n] = t
    captures = [c for c in captures if not isinstance(c, DirectCapture)]
    shapes = {}
    for c in captures:
        shapes[f"{c.name}.weight"] = (c.G.shape[-1], c.A.shape[-1])
        if c.has_bias:
            shapes[f"{c.name}.bias"] = (c.G.shape[-1],)
    if len(shapes) != sum(1 + c.has_bias for c in captures):
        raise ConfigurationError("layer names must be unique")
    for n, t in direct.items():
        if n in shapes:
            raise ConfigurationError(f"leaf {n!r} is given twice")
        shapes[n] = tuple(t.shape[1:])
    if not shapes:
        raise ConfigurationError("no layers to clip")
    leaf_names = sorted(shapes)
    leaf_index = {n: i for i, n in enumerate(leaf_names)}
    leaf_group, group_names, bounds = _groups_of(leaf_names, clipping_norm)
    n_groups = len(bounds)

    B = None
    dense, segmented = [], []
    direct_jobs = {}
    for c in captures:
        g = leaf_group[f"{c.name}.weight"]
        if c.has_bias and leaf_group[f"{c.name}.bias"] != g:
            raise ConfigurationError(
                f"layer {c.name!r}: weight and bias must be in the same clipping group")
        G = c.G if c.G.dtype == c.A.dtype else c.G.to(c.A.dtype)
        if c.norm_method not in ("auto", "gram", "direct"):
            raise ConfigurationError(f"layer {c.name!r}: unknown norm_method {c.norm_method!r}")
        if c.segments is None:
            nb = c.A.shape[0]
            if B is None:
                B = nb
            A3, G3 = _as_btd(c.A, B), _as_btd(G, B)
            if A3.shape[1] != G3.shape[1]:
                raise ConfigurationError(f"layer {c.name!r}: A and G disagree on the token count")
            T_, din_, dout_ = A3.shape[1], A3.shape[2], G3.shape[2]
            direct_ok = min(din_, dout_) <= ops.NARROW_MAX and T_ > 1
            if c.norm_method == "direct" and not direct_ok:
                raise ConfigurationError(
                    f"layer {c.name!r}: the direct method needs din or dout <= {ops.NARROW_MAX}")
            if direct_ok and (c.norm_method == "direct" or (
                    c.norm_method == "auto" and _direct_is_cheaper(T_, din_, dout_))):
                # Materialised per-example gradients, clipped as leaves (formed
                # below, the layers of one dtype and shape class together).
                pdt = c.param_dtype or A3.dtype
                direct_jobs.setdefault((A3.dtype, pdt, T_), []).append((c.name, A3, G3))
                if c.has_bias:
                    direct[f"{c.name}.bias"] = G3.float().sum(dim=1).to(pdt)
                continue
            dense.append(_Layer(c, g, A3.contiguous(), G3.contiguous()))
        else:
            if c.has_bias:
                raise ConfigurationError(
                    f"layer {c.name!r}: row-segmented layers with a bias are not supported")
            A2 = c.A.reshape(-1, c.A.shape[-1]).contiguous()
            G2 = G.reshape(-1, G.shape[-1]).contiguous()
            if B is None:
                B = len(c.segments)
            if len(c.segments) != B or sum(c.segments) != A2.shape[0] or G2.shape[0] != A2.shape[0]:
                raise ConfigurationError(
                    f"layer {c.name!r}: the row segments must give B row counts that add up "
                    "to the layer's input rows")
            segmented.append(_Layer(c, g, A2, G2))
    for (_, pdt, _), jobs in direct_jobs.items():
        ev = _event_pair(gemm_events)
        grads = ops.per_example_grads_grouped([A3 for _, A3, _ in jobs], [G3 for _, _, G3 in jobs],
                                              out_dtype=pdt)
        _close_pair(ev)
        for (name, _, _), g in zip(jobs, grads):
            direct[f"{name}.weight"] = g
    direct_names = sorted(direct)
    if direct_names:
        nb = direct[direct_names[0]].shape[0]
        if B is None:
            B = nb
        if any(direct[n].shape[0] != B for n in direct_names):
            raise ConfigurationError("the per-example gradients do not share the batch size")
    device = (dense + segmented)[0].A.device if (dense or segmented) else \
        direct[direct_names[0]].device

    # Per-group, per-example squared norms and the bounds of their rounding
    # errors (the ghost norms' sq + err bounds ||g||^2; the materialised
    # leaves' norms follow the reference's own roundoff, in the guard).
    sq_err = torch.zeros((2, n_groups, B), dtype=torch.float64, device=device)
    sq, err = sq_err[0], sq_err[1]
    gram_batches = {}
    for L in dense:
        if L.A.shape[1] == 1:
            ops.flat_sqnorms(L.A[:, 0], L.G[:, 0], with_bias=L.cap.has_bias, out=sq[L.group],
                             err=err[L.group])
        elif L.cap.has_bias:
            ops.gram_sqnorms(L.A, L.G, with_bias=True, out=sq[L.group], err=err[L.group])
        else:
            gram_batches.setdefault((L.group, L.A.dtype, L.A.shape[1]), []).append(L)
    # Bias-free layers of one clipping group, dtype and token count: one Gram
    # launch for all of them (up to 8 layers each).
    for (g, _, _), members in gram_batches.items():
        for k in range(0, len(members), 8):
            part = members[k:k + 8]
            if len(part) == 1:
                ops.gram_sqnorms(part[0].A, part[0].G, out=sq[g], err=err[g])
            else:
                ops.gram_sqnorms_multi([L.A for L in part], [L.G for L in part], out=sq[g],
                                       err=err[g])
    # The norms of all segmented layers of one dtype in one grouped launch
    # (up to 64 layers each; mixed shapes, most expensive tile pairs first).
    by_dtype = {}
    for L in segmented:
        by_dtype.setdefault(L.A.dtype, []).append(L)
    cap = ops.SegmentLayout.MAX_GRAM_PROBLEMS
    for members_all in by_dtype.values():
        for c0 in range(0, len(members_all), cap):
            members = members_all[c0:c0 + cap]
            layout = ops.SegmentLayout([L.cap.segments for L in members], device,
                                       gram_weights=[L.A.shape[1] + L.G.shape[1] for L in members],
                                       gram_dims=[(L.A.shape[1], L.G.shape[1]) for L in members])
            seg_sq, seg_err = ops.grouped_gram_sqnorms(
                [L.A for L in members], [L.G for L in members], layout, return_error=True)
            # Per-group sums over the layers, in layer order: the [E, B]
            # columns folded by group and added to the group's running sums.
            cols = device_table([L.group for L in members], np.int32, device)
            for acc, per_seg in ((sq, seg_sq), (err, seg_err)):
                per_seg = per_seg.contiguous()
                nat.call("dpc_group_sum_f64", nat.ptr(per_seg), B, len(members), 1, B,
                         nat.ptr(cols), n_groups, nat.ptr(acc), 1, nat.stream_handle(device))
    # The clipped sums: one grouped launch per layer shape.
    buckets = {}
    for L in segmented:
        buckets.setdefault((L.A.shape[1], L.G.shape[1], L.A.dtype), []).append(L)
    bucket_layouts = [(members, ops.SegmentLayout([L.cap.segments for L in members], device))
                      for members in buckets.values()]

    # Materialised per-example gradients: per-leaf squared norms, summed into
    # their groups in leaf order.
    direct_batch = None
    if direct_names:
        direct_batch = LeafBatch([direct[n].detach() for n in direct_names])
        leaf_sq = direct_batch.sqnorms()
        cols = [leaf_group[n] for n in direct_names]
        col_group = device_table(cols, np.int32, device)
        nat.call("dpc_group_sum_f64", nat.ptr(leaf_sq), B, len(cols), len(cols), 1,
                 nat.ptr(col_group), n_groups, nat.ptr(sq), 1, nat.stream_handle(device))

    # Guards for the materialised leaves the reference would clip.
    sizes = [math.prod(shapes[n]) for n in leaf_names]
    roundoff = num.norm_roundoff(torch.float32, torch.float64, len(sizes),
                                 num.reduction_terms(sizes))
    storage = sorted({L.A.dtype for L in dense + segmented} | {direct[n].dtype for n in direct},
                     key=str)
    guards = [num.guard_constants(dt, torch.promote_types(dt, torch.float32), roundoff)
              for dt in storage]
    # Only Gram and flat norms can come out non-finite (materialised
    # per-example gradients are sanitised by the leaf kernels), so a step of
    # direct layers alone never waits for its norm pass on the host.
    _nf.check_mode(nonfinite)
    watch = _nf.watch(device, n_groups, nonfinite) if dense or segmented else None
    # Every group's clip factors in one launch (group g: row g of each output).
    cfg = ops.clip_factors_groups(
        sq, [num.conservative_bound(bounds[g]) for g in range(n_groups)], guards, err=err,
        kind=kind, gamma=gamma, count_thresholds=[num.float32_of(b) for b in bounds],
        nonfinite=watch.flags if watch is not None else None)
    cfs = [cfg.group(g) for g in range(n_groups)]

    std = 0.0
    gen = None
    step_key = None
    next_noise_state = None
    if noise_fn is not None:
        if noise_state is None:
            raise ConfigurationError("noise_state is required with noise_fn")
        std = noise_fn.clipped_stddev(clipped(None, max_norm=max_norm))
        noisy = any((std.for_path(param_path(n)) if isinstance(std, PerGroup) else std) != 0.0
                    for n in leaf_names)
        step_key = step_key_for(noise_state)
        if noisy and noise_fn.stream == "reference":
            gen = generator_from_key(step_key)
        next_noise_state = GaussianNoiseState(
            _step_counter=noise_state._step_counter + 1, _rng_key=noise_state._rng_key)

    def leaf_std(leaf: str) -> float:
        if noise_fn is None:
            return 0.0
        if isinstance(std, PerGroup):
            return float(std.for_path(param_path(leaf)))
        return float(std)

    # Reference-stream draws: one generator, flatten order, no draw for a
    # leaf whose standard deviation is 0.
    draws = {}
    if gen is not None:
        for leaf in leaf_names:
            if leaf_std(leaf) != 0.0:
                draws[leaf] = torch.randn(shapes[leaf], dtype=torch.float32, generator=gen)

    def to_dev(t):
        return t.pin_memory().to(device, non_blocking=True)

    tree = {}
    multi = {}
    for L in dense:
        si = storage.index(L.A.dtype)
        cf = cfs[L.group]
        wn, bn = f"{L.name}.weight", f"{L.name}.bias"
        spec = None
        s_w = leaf_std(wn)
        s_b = leaf_std(bn) if L.cap.has_bias else s_w
        if s_w != s_b:
            raise ConfigurationError(
                f"layer {L.name!r}: weight and bias noise must share a standard deviation")
        if s_w != 0.0:
            if gen is not None:
                spec = ops.NoiseSpec(
                    sigma=s_w, mode=nat.NOISE_INJECTED, noise=to_dev(draws[wn]),
                    bias_noise=to_dev(draws[bn]) if L.cap.has_bias else None)
            else:
                spec = ops.NoiseSpec(sigma=s_w, mode=nat.NOISE_PHILOX, seed=step_key.seed,
                                     leaf_id=leaf_index[wn], bias_leaf_id=leaf_index.get(bn, 0))
        out_dtype = dtype or L.cap.param_dtype or L.A.dtype
        if L.cap.has_bias:
            ev = _event_pair(gemm_events)
            w, b = ops.clipped_sum(L.A, L.G, cf.scale[si], plan=cf.plan[si],
                                   normalize_by=normalize_by, noise=spec, out_dtype=out_dtype,
                                   with_bias=True)
            _close_pair(ev)
            tree[wn] = w
            tree[bn] = b
            continue
        # Bias-free layers of one clipping group, operand dtype, output dtype
        # and noise kind go out together (their output tiles share launches).
        kind = (spec.mode, spec.seed) if spec is not None else None
        multi.setdefault((L.group, si, L.A.dtype, out_dtype, kind), []).append((L, wn, spec))
    for (g, si, _, out_dtype, _), members in multi.items():
        cf = cfs[g]
        ev = _event_pair(gemm_events)
        if len(members) == 1:
            L, wn, spec = members[0]
            outs = [ops.clipped_sum(L.A, L.G, cf.scale[si], plan=cf.plan[si],
                                    normalize_by=normalize_by, noise=spec,
                                    out_dtype=out_dtype)[0]]
        else:
            outs = ops.clipped_sum_multi([L.A for L, _, _ in members],
                                         [L.G for L, _, _ in members], cf.scale[si],
                                         plan=cf.plan[si], normalize_by=normalize_by,
                                         noises=[sp for _, _, sp in members],
                                         out_dtype=out_dtype)
        _close_pair(ev)
        for (_, wn, _), w in zip(members, outs):
            tree[wn] = w
    for members, layout in bucket_layouts:
        si = storage.index(members[0].A.dtype)
        seg_scale = _group_rows(cfg.scale, [L.group for L in members], si)
        names = [f"{L.name}.weight" for L in members]
        sigmas = [leaf_std(n) for n in names]
        gnoise = None
        if any(s != 0.0 for s in sigmas):
            if gen is not None:
                zero = None
                noise = []
                for n in names:
                    if n in draws:
                        noise.append(to_dev(draws[n]))
                    else:
                        if zero is None:
                            zero = torch.zeros(shapes[n], dtype=torch.float32, device=device)
                        noise.append(zero)
                gnoise = ops.GroupedNoise(sigmas=sigmas, mode=nat.NOISE_INJECTED, noise=noise)
            else:
                gnoise = ops.GroupedNoise(sigmas=sigmas, mode=nat.NOISE_PHILOX, seed=step_key.seed,
                                          leaf_ids=[leaf_index[n] for n in names])
        out_dtype = dtype or members[0].cap.param_dtype or members[0].A.dtype
        ev = _event_pair(gemm_events)
        stacked = ops.grouped_clipped_sum([L.A for L in members], [L.G for L in members], layout,
                                          seg_scale, normalize_by=normalize_by, noise=gnoise,
                                          out_dtype=out_dtype)
        _close_pair(ev)
        for i, n in enumerate(names):
            tree[n] = stacked[i]
    if direct_batch is not None:
        scale_rows = {dt: _group_rows(cfg.scale, list(range(n_groups)), storage.index(dt))
                      for dt in direct_batch.dtypes}
        sum_dtypes = ({dt: (_sum_dtype_of(dt, None), dtype) for dt in direct_batch.dtypes}
                      if dtype is not None else None)
        reduced, _ = direct_batch.apply(scale_rows, [leaf_group[n] for n in direct_names],
                                        sum_dtypes)
        philox = {}
        for n, x in zip(direct_names, reduced):
            if normalize_by != 1.0:
                x = x / normalize_by
            s_n = leaf_std(n)
            if s_n != 0.0:
                if gen is not None:
                    x = ops.add_noise(x, s_n, mode=nat.NOISE_INJECTED, noise=to_dev(draws[n]))
                else:
                    # Added below, in place (x is this step's own buffer), the
                    # leaves of one dtype in one launch.
                    philox.setdefault(x.dtype, []).append((n, x, s_n))
            tree[n] = x
        for items in philox.values():
            ops.add_noise_leaves([x for _, x, _ in items], [s for _, _, s in items],
                                 seed=step_key.seed, leaf_ids=[leaf_index[n] for n, _, _ in items],
                                 inplace=True)
    tree = {k: tree[k] for k in leaf_names}
    if watch is not None and watch.count() > 0:
        _clip_nonfinite_examples(
            dense, segmented, direct, leaf_names, leaf_group, bounds, sq, err, cfs, storage, tree,
            per_group=per_group, kind=kind, gamma=gamma, normalize_by=normalize_by, dtype=dtype)
    if noise_fn is None:
        result = clipped(tree, max_norm=max_norm)
    else:
        result = NoisedPytree(pytree=tree, max_norm=max_norm, noise_stddev=std)
    if return_aux:
        total = sq.sum(dim=0) if n_groups > 1 else sq[0]
        group_norms = None
        if per_group:
            group_norms = {n: cfs[k].norms for k, n in enumerate(group_names)}
        aux = GhostGradAux(
            loss_values=None,
            grad_norms=torch.sqrt(total).to(torch.float32) if per_group else cfs[0].norms,
            clip_scales=cfg.scale if per_group else cfs[0].scale,
            num_clipped=cfg.nclipped,
            batch_size=B, group_norms=group_norms)
        result = (result, aux)
    if noise_fn is None:
        return result
    return result, next_noise_state


def _group_rows(scale: torch.Tensor, groups: list[int], guard: int) -> torch.Tensor:
    """Rows ``scale[g, guard]`` for g in ``groups`` ([len(groups), B], contiguous):
    a view when they are all the groups in order and the guard's rows are
    contiguous, else a gather."""
    G = scale.shape[0]
    if groups == list(range(G)) and (scale.shape[1] == 1 or G == 1):
        return scale[:, guard]
    return scale[:, guard].index_select(0, device_table(groups, np.int32, scale.device))


def _scale_kind(auto_s_gamma):
    if auto_s_gamma is None:
        return nat.SCALE_FIXED, 0.0
    if isinstance(auto_s_gamma, bool) or not auto_s_gamma > 0:
        raise ConfigurationError(f"gamma must be positive, got {auto_s_gamma}")
    return nat.SCALE_AUTO_S, float(auto_s_gamma)


def _clip_nonfinite_examples(dense, segmented, direct, leaf_names, leaf_group, bounds, sq, err,
                             cfs, storage, tree, *, per_group, kind, gamma, normalize_by, dtype):
    """The (example, group) pairs whose norm is not finite (a dense or
    segmented layer of the group holds NaN/Inf for the example), clipped from
    the example's sanitised per-example gradients of that group's leaves --
    as the reference materialises them -- by the leaf kernels with the
    group's bound; their sums are added to ``tree`` and their norms, scales
    and counts replace the flagged entries in ``sq`` / ``cfs``.  A group's
    clip factor depends on that group's leaves only, so pairs whose group
    norm is finite were already right."""
    scale = "auto_s" if kind == nat.SCALE_AUTO_S else "fixed"
    for g, cf in enumerate(cfs):
        bad = _nf.bad_examples(sq[g], err[g])
        if bad.numel() == 0:
            continue
        bad_list = bad.tolist()
        names = [n for n in leaf_names if leaf_group[n] == g]
        leaves = {}
        for L in dense:
            wn, bn = f"{L.name}.weight", f"{L.name}.bias"
            if wn not in names and bn not in names:
                continue
            pdt = L.cap.param_dtype or L.A.dtype
            w, b = _nf.sanitized_linear_grads(L.A[bad], L.G[bad], pdt, L.cap.has_bias)
            leaves[wn] = w
            if b is not None:
                leaves[bn] = b
        for L in segmented:
            wn = f"{L.name}.weight"
            if wn not in names:
                continue
            pdt = L.cap.param_dtype or L.A.dtype
            starts = np.concatenate([[0], np.cumsum(L.cap.segments)]).tolist()
            ws = []
            for b in bad_list:
                r0, r1 = starts[b], starts[b + 1]
                if r1 == r0:
                    ws.append(torch.zeros((L.G.shape[1], L.A.shape[1]), dtype=pdt,
                                          device=L.A.device))
                    continue
                w, _ = _nf.sanitized_linear_grads(L.A[r0:r1].unsqueeze(0),
                                                  L.G[r0:r1].unsqueeze(0), pdt, False)
                ws.append(w[0])
            leaves[wn] = torch.stack(ws)
        for n, t in direct.items():
            if n in names:
                leaves[n] = t[bad]
        order = [leaves[n] for n in names]
        sum_dtypes = {t.dtype: (_sum_dtype_of(t.dtype, None), dtype or t.dtype) for t in order}
        res = leaves_clip_sum(order, bounds[g], kind=scale, gamma=gamma, sum_dtypes=sum_dtypes)
        for n, x in zip(names, res.reduced):
            if normalize_by != 1.0:
                x = x / normalize_by
            tree[n] = (tree[n] + x).to(tree[n].dtype)
        cf.norms[bad] = res.norms.to(cf.norms.dtype)
        for si, dt in enumerate(storage):
            if dt in res.scales:
                cf.scale[si][bad] = res.scales[dt][0]
        cf.nclipped.copy_((cf.norms > num.float32_of(bounds[g])).sum().reshape(1).to(torch.int32))
        sq[g, bad] = res.norms.double() ** 2
        err[g, bad] = 0.0


def _capture(model, layers, others, loss_fn, inputs, targets):
    hooks = [_Capture(mod) for _, mod in layers]
    dhooks = [_DirectHook(mod) for _, mod, _ in others]
    args = inputs if isinstance(inputs, tuple) else (inputs,)
    try:
        with record_function("opake::ghost_capture"), torch.enable_grad():
            outputs = model(*args)
            losses = loss_fn(outputs, targets)
            if losses.dim() != 1:
                raise ConfigurationError("loss_fn must return per-example losses [B]")
            named = [(n, c) for (n, _), c in zip(layers, hooks)]
            named += [(n, c) for (n, _, _), c in zip(others, dhooks)]
            for name, cap in named:
                if cap.out is None:
                    raise ConfigurationError(f"module {name!r} was not used by the forward pass")
                if cap.calls != 1:
                    raise ConfigurationError(
                        f"module {name!r} was called {cap.calls} times; ghost clipping needs "
                        "one call per module and step")
            # Gradients with respect to the module outputs only: autograd
            # prunes the weight-gradient GEMMs, which the clipped sum replaces.
            grads = torch.autograd.grad(losses.sum(), [c.out for _, c in named],
                                        allow_unused=True)
    finally:
        for c in hooks + dhooks:
            c.remove()
    B = losses.shape[0]
    captures = []
    for (name, mod), cap, g in zip(layers, hooks, grads[:len(layers)]):
        G = g.detach() if g is not None else torch.zeros_like(cap.out)
        if cap.segments is None and cap.A.shape[0] != B:
            raise ConfigurationError(
                f"layer {name!r}: its input does not have the batch as dim 0 (a layer fed "
                "with the rows of several examples must set dpc_row_segments)")
        captures.append(LinearCapture(name=name, A=cap.A, G=G, has_bias=mod.bias is not None,
                                      segments=cap.segments, param_dtype=mod.weight.dtype))
        cap.out = None
    per_ex = {}
    for (name, mod, own), cap, g in zip(others, dhooks, grads[len(layers):]):
        G = g.detach() if g is not None else torch.zeros_like(cap.out)
        if G.shape[0] != B:
            raise ConfigurationError(f"module {name!r}: its output does not have the batch "
                                     "as dim 0")
        with torch.enable_grad():
            pg = _per_example_param_grads(mod, own, cap.args, G)
        for pn, t in pg.items():
            per_ex[f"{name}.{pn}" if name else pn] = t.detach()
        cap.out = None
    if per_ex:
        captures.append(DirectCapture(per_ex))
    return captures, losses.detach()


def ghost_capture(model: torch.nn.Module, loss_fn, inputs, targets):
    """One forward of ``model`` and the backward to its trainable modules'
    outputs: the operands ghost clipping needs, without clipping them.

    Returns ``(captures, losses)``: a :class:`LinearCapture` per linear layer
    and one :class:`DirectCapture` with the materialised per-example gradients
    of the other trainable parameters; ``ghost_clip_captured(captures, ...)``
    then gives ``ghost_clipped_grad``'s result.
    """
    layers, others = _trainable_modules(model)
    return _capture(model, layers, others, loss_fn, inputs, targets)


def _slice_batch(x, start, stop):
    if isinstance(x, tuple):
        return tuple(_slice_batch(v, start, stop) for v in x)
    return x[start:stop] if isinstance(x, torch.Tensor) else x


def _merge_aux(parts):
    group_norms = None
    if parts[0].group_norms is not None:
        group_norms = {k: torch.cat([p.group_norms[k] for p in parts]) for k in parts[0].group_norms}
    return GhostGradAux(
        loss_values=torch.cat([p.loss_values for p in parts]),
        grad_norms=torch.cat([p.grad_norms for p in parts]),
        clip_scales=torch.cat([p.clip_scales for p in parts], dim=-1),
        num_clipped=torch.stack([p.num_clipped for p in parts]).sum(dim=0),
        batch_size=sum(p.batch_size for p in parts),
        group_norms=group_norms)


def ghost_clipped_grad(
    model: torch.nn.Module,
    loss_fn,
    *,
    clipping_norm,
    normalize_by: float = 1.0,
    return_aux: bool = False,
    dtype: torch.dtype | None = None,
    microbatch_size: int | None = None,
    auto_s_gamma: float | None = None,
    nonfinite: str = "sanitize",
):
    """Create ``grad_fn(inputs, targets, *, state, noise_fn=None, noise_state=None)``.

    ``loss_fn(outputs, targets)`` must return per-example losses ``[B]``
    (e.g. ``cross_entropy(..., reduction="none")``).  ``inputs`` is one tensor
    or a tuple of positional arguments of ``model``.  Without ``noise_fn`` the
    call returns ``(ClippedPytree, state)``; with it, ``(NoisedPytree, state,
    noise_state')`` where the noise was fused into the clipped-sum epilogue.
    With ``return_aux`` the first element is ``(result, GhostGradAux)``.

    ``microbatch_size`` runs the forward, backward and clipped sum chunk by
    chunk (chunk sums accumulated in float32 and cast once, as
    ``_microbatch_accumulate_reduced``, _clipped_fun.py:252-345); the noise is
    then added to the total by ``noise_fn`` (not fused).

    ``auto_s_gamma``: AUTO-S scaling (``auto_clipped_grad``, _auto.py:211-367)
    with ``R = clipping_norm``; ``nonfinite``: as in
    :func:`ghost_clip_captured`.
    """
    _validate_bound(clipping_norm)
    _scale_kind(auto_s_gamma)
    _nf.check_mode(nonfinite)
    if normalize_by <= 0.0:
        raise ConfigurationError(f"normalize_by must be > 0, got {normalize_by}.")
    if microbatch_size is not None and (isinstance(microbatch_size, bool)
                                        or not isinstance(microbatch_size, int)
                                        or microbatch_size <= 0):
        raise ConfigurationError(f"microbatch_size must be a positive int, got {microbatch_size}")
    layers, others = _trainable_modules(model)
    leaf_names = []
    for name, mod in layers:
        leaf_names.append(f"{name}.weight")
        if mod.bias is not None:
            leaf_names.append(f"{name}.bias")
    for name, _, own in others:
        leaf_names.extend(f"{name}.{pn}" if name else pn for pn, _ in own)
    _groups_of(leaf_names, clipping_norm)  # validates a PerGroup against the leaves
    state0 = FixedClipState()

    def microbatched(inputs, targets, *, state, noise_fn=None, noise_state=None):
        B = targets.shape[0]
        acc, auxes, max_norm = None, [], None
        for start in range(0, B, microbatch_size):
            stop = min(B, start + microbatch_size)
            captures, losses = _capture(model, layers, others, loss_fn,
                                        _slice_batch(inputs, start, stop), targets[start:stop])
            out = ghost_clip_captured(captures, clipping_norm=clipping_norm,
                                      normalize_by=normalize_by, dtype=torch.float32,
                                      return_aux=return_aux, auto_s_gamma=auto_s_gamma,
                                      nonfinite=nonfinite)
            if return_aux:
                out, aux = out
                auxes.append(replace(aux, loss_values=losses.detach()))
            max_norm = out.max_norm
            acc = out.pytree if acc is None else {k: acc[k] + v for k, v in out.pytree.items()}
        param_dtype = {n: p.dtype for n, p in model.named_parameters()}
        tree = {k: v.to(dtype or param_dtype.get(k, v.dtype)) for k, v in acc.items()}
        result = clipped(tree, max_norm=max_norm)
        next_state = None
        if noise_fn is not None:
            if noise_state is None:
                raise ConfigurationError("noise_state is required with noise_fn")
            result, next_state = noise_fn(result, noise_state)
        if return_aux:
            result = (result, _merge_aux(auxes))
        if noise_fn is None:
            return result, state
        return result, state, next_state

    def grad_fn(inputs, targets, *, state, noise_fn=None, noise_state=None):
        if microbatch_size is not None and targets.shape[0] > microbatch_size:
            return microbatched(inputs, targets, state=state, noise_fn=noise_fn,
                                noise_state=noise_state)
        captures, losses = _capture(model, layers, others, loss_fn, inputs, targets)
        out = ghost_clip_captured(captures, clipping_norm=clipping_norm,
                                  normalize_by=normalize_by, noise_fn=noise_fn,
                                  noise_state=noise_state, dtype=dtype, return_aux=return_aux,
                                  auto_s_gamma=auto_s_gamma, nonfinite=nonfinite)
        if noise_fn is not None:
            out, next_state = out
        if return_aux:
            result, aux = out
            out = (result, replace(aux, loss_values=losses.detach()))
        if noise_fn is None:
            return out, state
        return out, state, next_state

    return grad_fn, state0


def auto_ghost_clipped_grad(
    model: torch.nn.Module,
    loss_fn,
    *,
    R=1.0,
    gamma: float = 0.01,
    normalize_by: float = 1.0,
    return_aux: bool = False,
    dtype: torch.dtype | None = None,
    microbatch_size: int | None = None,
    nonfinite: str = "sanitize",
):
    """:func:`ghost_clipped_grad` with AUTO-S scaling ``R / (||g_i|| + gamma)``
    (``auto_clipped_grad``, _auto.py:211-367): ``max_norm = R /
    normalize_by``; ``R`` may be a ``PerGroup``."""
    return ghost_clipped_grad(model, loss_fn, clipping_norm=R, normalize_by=normalize_by,
                              return_aux=return_aux, dtype=dtype,
                              microbatch_size=microbatch_size, auto_s_gamma=gamma,
                              nonfinite=nonfinite)


__all__ = [
    "auto_ghost_clipped_grad",
    "DirectCapture",
    "GhostGradAux",
    "LinearCapture",
    "ghost_capture",
    "ghost_clip_captured",
    "ghost_clipped_grad",
]
