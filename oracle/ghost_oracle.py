"""Materialised per-example gradients on the CPU (the reference's ``vmap(grad)``).

TEST INFRASTRUCTURE: imported only by tests/, smoke() and bench.py's CPU
baseline.

The reference computes per-example gradients with
``torch.func.vmap(grad_and_value(loss_fn))``
(packages/opake-engine/src/opake/api/engine/clipping/_clipped_grad.py:278-296,
_clipped_fun.py:476-489).  For a linear layer y = x W^T (+ b) with output
gradient G the per-example weight gradient is G_i^T A_i and the bias gradient
sum_t G_i[t]; the linear surrogate loss L_i(W) = sum_t <G_i[t], W A_i[t]> of the
benchmark configuration has exactly this gradient.
"""

from __future__ import annotations

import torch
from torch.func import functional_call, grad, vmap


def linear_per_example_grads(A: torch.Tensor, G: torch.Tensor, *, dtype=None,
                             with_bias: bool = False):
    """Per-example weight (and bias) gradients of a linear layer.

    Computed in float64 from the given values and rounded once to ``dtype``
    (default: the input dtype) -- the value a per-example backward stores.
    Returns a list of stacked leaves in the sorted key order of
    ``{"bias", "weight"}``.
    """
    dtype = dtype or A.dtype
    w = torch.einsum("btm,btn->bmn", G.double(), A.double()).to(dtype)
    if not with_bias:
        return [w]
    b = G.double().sum(dim=1).to(dtype)
    return [b, w]


def surrogate_per_example_grads(A: torch.Tensor, G: torch.Tensor):
    """The reference path literally: vmap(grad) of the surrogate loss."""
    dout, din = G.shape[2], A.shape[2]
    W = torch.zeros(dout, din, dtype=A.dtype)

    def loss(w, a, g):
        return (g * (a @ w.T)).sum()

    return vmap(grad(loss), in_dims=(None, 0, 0))(W, A, G)


class MLP(torch.nn.Module):
    """The config-1 model: 784-512-10 with ReLU."""

    def __init__(self, d_in=784, d_hidden=512, d_out=10):
        super().__init__()
        self.fc1 = torch.nn.Linear(d_in, d_hidden)
        self.fc2 = torch.nn.Linear(d_hidden, d_out)

    def forward(self, x):
        return self.fc2(torch.relu(self.fc1(x)))


def mlp_per_example_grads(model: torch.nn.Module, params: dict, x: torch.Tensor,
                          y: torch.Tensor) -> dict:
    """vmap(grad) of the per-example cross-entropy, as the reference runs it."""

    def loss_fn(p, xb, yb):
        logits = functional_call(model, p, (xb.unsqueeze(0),))
        return torch.nn.functional.cross_entropy(logits, yb.unsqueeze(0))

    return vmap(grad(loss_fn), in_dims=(None, 0, 0))(params, x, y)


def segment_grads(A: torch.Tensor, G: torch.Tensor, lengths, *, dtype=None) -> torch.Tensor:
    """Per-segment weight gradients of a row-segmented linear layer.

    ``A`` [rows, din], ``G`` [rows, dout]; ``lengths`` are the consecutive
    segments' row counts.  Segment v's gradient is ``G_v^T A_v`` over its rows
    (the per-sample gradient of a "virtual expert", the reference's
    ``_grouped_AtB`` out[g] = A_g^T B_g,
    packages/opake-patches/src/opake/api/patches/kernels/fused_moe.py:54-113),
    computed in float64 and rounded once to ``dtype``.  Returns [S, dout, din].
    """
    dtype = dtype or A.dtype
    out = torch.zeros(len(lengths), G.shape[1], A.shape[1], dtype=torch.float64)
    start = 0
    for v, n in enumerate(lengths):
        if n:
            out[v] = G[start:start + n].double().T @ A[start:start + n].double()
        start += n
    return out.to(dtype)


def per_example_grads_loop(model: torch.nn.Module, loss_fn, args: tuple, targets,
                           batch_args=None) -> dict:
    """Per-example gradients of every trainable parameter by brute force: one
    forward and backward of ``model`` per example on its own slice.

    ``loss_fn(outputs, targets)`` returns per-example losses; ``batch_args``
    marks which positional args carry the batch (default: all).  Returns
    ``{parameter name: [B, *shape]}`` in float64 of the parameter values.
    """
    params = {n: p for n, p in model.named_parameters() if p.requires_grad}
    B = targets.shape[0]
    batch_args = batch_args or tuple(range(len(args)))
    out = {n: [] for n in params}
    for i in range(B):
        sl = tuple(a[i:i + 1] if j in batch_args else a for j, a in enumerate(args))
        loss = loss_fn(model(*sl), targets[i:i + 1]).sum()
        gs = torch.autograd.grad(loss, list(params.values()), allow_unused=True)
        for (n, p), g in zip(params.items(), gs):
            out[n].append(torch.zeros_like(p) if g is None else g.detach())
    return {n: torch.stack(v) for n, v in out.items()}


__all__ = [
    "MLP",
    "per_example_grads_loop",
    "segment_grads",
    "linear_per_example_grads",
    "mlp_per_example_grads",
    "surrogate_per_example_grads",
]
