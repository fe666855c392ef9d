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


# --- the error bound of the Gram norm ------------------------------------------
#
# The ghost norm <A A^T, G G^T> cancels, so the device returns an upper bound
# `err` of its rounding error with every squared norm (the clip factor is taken
# from sq + err).  The bound is new work of this build -- the reference
# materialises gradients and has no Gram norm -- so the functions below restate
# the device formula (opake_amd/csrc/common.h: dpc_chain_gamma, dpc_row_bound;
# opake_amd/csrc/gram.hip: the tile records and gram_bound_wave) for the CPU
# tests, which pin it by its defining property
# |S - ||g||^2| <= err on emulated accumulation chains of the two rounding
# behaviours the model covers (round-to-nearest, truncation) and on crafted
# cancellation inputs, with exact float64 gradients as the truth.

U_MFMA = 2.0 ** -23
U_FP64 = 2.0 ** -52
ROW_SLACK_MFMA = 2.0 ** -51


def chain_gamma(n: float, u: float) -> float:
    """gamma(n) = g / (1 - g), g = (18/16) n u, rounded up by 2^-40."""
    g = 1.125 * n * u
    if not g < 0.5:
        return float("inf")
    return g / (1.0 - g) * (1.0 + 2.0 ** -40)


def row_bound(diag: float, gamma: float, eta: float, slack: float) -> float:
    """Upper bound of ||a_s|| + slack from the computed diagonal entry P^_ss."""
    inv = (1.0 + 2.0 ** -50) / (1.0 - gamma)
    return (abs(diag) + eta) ** 0.5 * inv ** 0.5 * (1.0 + 2.0 ** -50) + slack


def gram_error_bound(P, Q, *, d_p: int, d_q: int, tile: int = 128, mfma: bool = True):
    """``(S, err)`` for one example from its computed Gram matrices.

    ``P`` / ``Q``: [T, T] Gram matrices (float64 arrays of the computed fp32
    values) of the operands of widths ``d_p`` / ``d_q``; the narrower one
    takes the role of P (as the kernel orders them).  ``S`` is the tile-wise
    inner product; ``err`` bounds ``|S - ||G^T A||^2|``:
      gA X + gQ Y + (gA gQ + g64 (1 + gA)(1 + gQ)) W2 V2,
    X = sum of the diagonal tiles' w_s^2 |Q_ss| and ||w_p||^2 ||Q_pp,off||_F,
    plus 2 ||w_p|| ||w_q|| ||Q_pq||_F over p < q; Y likewise with v and P.
    """
    import numpy as np

    P = np.asarray(P, dtype=np.float64)
    Q = np.asarray(Q, dtype=np.float64)
    if d_p > d_q:
        P, Q, d_p, d_q = Q, P, d_q, d_p
    T = P.shape[0]
    kstep = 32 if mfma else 16
    n_p = -(-d_p // kstep) * kstep
    n_q = -(-d_q // kstep) * kstep
    u = U_MFMA if mfma else U_FP64
    gA, gQ = chain_gamma(n_p, u), chain_gamma(n_q, u)
    etaA = n_p * 2.0 ** -125 if mfma else 0.0
    etaQ = n_q * 2.0 ** -125 if mfma else 0.0
    slack = ROW_SLACK_MFMA if mfma else 0.0
    nt = -(-T // tile)
    blocks = [slice(b * tile, min(T, (b + 1) * tile)) for b in range(nt)]
    W2 = np.zeros(nt)
    V2 = np.zeros(nt)
    S = 0.0
    X = Y = 0.0
    # Rows past T inside the last tile read as zero on the device: their
    # diagonal entries are 0 and still carry the slack weight.
    pad = nt * tile - T
    w_pad = row_bound(0.0, gA, etaA, slack) ** 2
    v_pad = row_bound(0.0, gQ, etaQ, slack) ** 2
    for b, sl in enumerate(blocks):
        dp, dq = np.diag(P[sl, sl]), np.diag(Q[sl, sl])
        ws = np.array([row_bound(x, gA, etaA, slack) for x in dp])
        vs = np.array([row_bound(x, gQ, etaQ, slack) for x in dq])
        W2[b] = (ws ** 2).sum() + (w_pad * pad if b == nt - 1 else 0.0)
        V2[b] = (vs ** 2).sum() + (v_pad * pad if b == nt - 1 else 0.0)
        X += (ws ** 2 * np.abs(dq)).sum()
        Y += (vs ** 2 * np.abs(dp)).sum()
    for q in range(nt):
        for p in range(q + 1):
            Pt, Qt = P[blocks[p], blocks[q]], Q[blocks[p], blocks[q]]
            inner = float((Pt * Qt).sum())
            if p == q:
                off = ~np.eye(Pt.shape[0], dtype=bool)
                S += inner
                X += W2[p] * float(((Qt * Qt)[off]).sum()) ** 0.5
                Y += V2[p] * float(((Pt * Pt)[off]).sum()) ** 0.5
            else:
                S += 2.0 * inner
                X += 2.0 * (W2[p] * W2[q] * float((Qt * Qt).sum())) ** 0.5
                Y += 2.0 * (V2[p] * V2[q] * float((Pt * Pt).sum())) ** 0.5
    g64 = (T * T + 256.0) * 2.0 ** -52
    err = gA * X + gQ * Y + (gA * gQ + g64 * (1 + gA) * (1 + gQ)) * W2.sum() * V2.sum()
    return S, err * (1.0 + 2.0 ** -40)


def emulated_gram(X, *, mode: str = "rn", block: int = 16):
    """``X X^T`` accumulated as an fp32 MFMA chain would: each block of
    ``block`` products (exact for bf16 inputs) summed in float64, then added
    to the fp32 accumulator; ``mode`` "rn" rounds both the block sum and the
    addition to nearest, "rz" truncates both toward zero.  float64 [T, T] of
    the fp32 results."""
    import numpy as np

    X = np.asarray(X, dtype=np.float64)
    T, d = X.shape

    def to_f32(v):
        r = v.astype(np.float32)
        if mode == "rz":
            away = np.abs(r.astype(np.float64)) > np.abs(v)
            r = np.where(away, np.nextafter(r, np.float32(0)), r)
        return r

    acc = np.zeros((T, T), dtype=np.float32)
    for k0 in range(0, d, block):
        Xb = X[:, k0:k0 + block]
        part = to_f32(Xb @ Xb.T)
        acc = to_f32(acc.astype(np.float64) + part.astype(np.float64))
    return acc.astype(np.float64)


__all__ = [
    "MLP",
    "chain_gamma",
    "emulated_gram",
    "gram_error_bound",
    "row_bound",
    "per_example_grads_loop",
    "segment_grads",
    "linear_per_example_grads",
    "mlp_per_example_grads",
    "surrogate_per_example_grads",
]
