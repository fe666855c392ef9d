"""Top-k mixture-of-experts SwiGLU FFN whose experts feed ghost clipping.

Forward semantics follow the reference's expert FFN
(packages/opake-patches/src/opake/api/patches/kernels/moe.py:74-103,
``opake_moe`` :570-627): per expert ``e``,
``h = silu(x W_gu[e][:I]^T) * (x W_gu[e][I:]^T)`` (the SiLU taken in float32
and cast back), ``y = h W_down[e]^T``, and each token's output is the
route-weighted sum over its top-k experts (accumulated in float32).  Routing
weights are the softmax over the top-k router logits.

Layout: each expert is its own module with two bias-free linear layers
(``experts.<e>.gate_up`` [2I, d] and ``experts.<e>.down`` [d, I]), so the
parameter pytree has one leaf per expert and projection and a ``PerGroup``
can put each expert in its own clipping group.  The router is a frozen
linear layer; ``forward`` also accepts router logits directly.

Dispatch sorts the (token, slot) assignments by expert and, within an
expert, by token, so expert ``e``'s input rows are its examples' tokens in
example order.  Before calling an expert's layers the module sets
``dpc_row_segments`` on them to the per-example row counts, which is what
the model-level ghost clipping needs to form per-example (per-expert) norms
and clipped sums without materialising a gradient.  Computing the counts
takes one device-to-host copy of the [E, B] count table per forward (the
per-expert GEMM shapes need it anyway).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn


class SwiGLUExpert(nn.Module):
    def __init__(self, d: int, inter: int, *, dtype=None, device=None):
        super().__init__()
        self.inter = inter
        self.gate_up = nn.Linear(d, 2 * inter, bias=False, dtype=dtype, device=device)
        self.down = nn.Linear(inter, d, bias=False, dtype=dtype, device=device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gu = self.gate_up(x)
        h = F.silu(gu[:, : self.inter].float()).to(x.dtype) * gu[:, self.inter:]
        return self.down(h)


class TopKMoE(nn.Module):
    """``d``-wide top-``k`` MoE FFN with ``n_experts`` SwiGLU experts of width ``inter``."""

    def __init__(self, d: int, inter: int, n_experts: int, top_k: int = 2, *, dtype=None,
                 device=None):
        super().__init__()
        if not 1 <= top_k <= n_experts:
            raise ValueError("top_k must be between 1 and n_experts")
        self.d, self.inter, self.n_experts, self.top_k = d, inter, n_experts, top_k
        self.router = nn.Linear(d, n_experts, bias=False, dtype=dtype, device=device)
        self.router.weight.requires_grad_(False)
        self.experts = nn.ModuleList(
            SwiGLUExpert(d, inter, dtype=dtype, device=device) for _ in range(n_experts))
        self.last_counts: torch.Tensor | None = None  # [E, B] host copy of the last routing

    def route(self, x: torch.Tensor, router_logits: torch.Tensor | None = None):
        """Top-k expert indices and weights ([B, T, k] each)."""
        logits = self.router(x) if router_logits is None else router_logits
        top_v, top_i = torch.topk(logits.float(), self.top_k, dim=-1)
        return top_i, torch.softmax(top_v, dim=-1).to(x.dtype)

    def forward(self, x: torch.Tensor, router_logits: torch.Tensor | None = None):
        B, T, d = x.shape
        E, k = self.n_experts, self.top_k
        top_i, top_w = self.route(x, router_logits)
        expert = top_i.reshape(-1)
        token = torch.arange(B * T, device=x.device).repeat_interleave(k)
        order = torch.argsort(expert * (B * T) + token, stable=True)
        counts = torch.bincount(expert * B + token // T, minlength=E * B).view(E, B).cpu()
        self.last_counts = counts
        rows = counts.sum(dim=1).tolist()
        tok_sorted = token[order]
        xs = x.reshape(B * T, d)[tok_sorted]
        outs = []
        start = 0
        for e in range(E):
            n = rows[e]
            mod = self.experts[e]
            seg = counts[e].tolist()
            mod.gate_up.dpc_row_segments = seg
            mod.down.dpc_row_segments = seg
            outs.append(mod(xs[start:start + n]))
            start += n
        y = torch.cat(outs) * top_w.reshape(-1)[order].unsqueeze(1)
        out = torch.zeros((B * T, d), dtype=torch.float32, device=x.device)
        out.index_add_(0, tok_sorted, y.float())
        return out.to(x.dtype).view(B, T, d)


def expert_groups(model: TopKMoE, prefix: str = "", clipping_norm: float = 1.0):
    """``PerGroup`` with one group per expert, ``C_e = C / sqrt(E)`` (so the
    effective bound is ``C``): the per-expert clipping of a MoE step."""
    import math

    from opake_amd.types import PerGroup

    groups, values = {}, {}
    bound = clipping_norm / math.sqrt(model.n_experts)
    for e in range(model.n_experts):
        name = f"expert{e}"
        values[name] = bound
        for proj in ("gate_up", "down"):
            groups[f"{prefix}experts.{e}.{proj}.weight"] = name
    return PerGroup(groups, values)


__all__ = ["SwiGLUExpert", "TopKMoE", "expert_groups"]
