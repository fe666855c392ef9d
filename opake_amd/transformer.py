"""A Llama-style transformer block for per-example clipping of its parameters.

Pre-norm block: RMSNorm -> causal multi-head self-attention with rotary
position embeddings -> residual -> RMSNorm -> SwiGLU FFN -> residual.  The
attention projections are one fused ``qkv`` linear layer (d -> 3d) and the FFN
input projections one fused ``gate_up`` layer (d -> 2F), so the layers that
share an input also share one Gram matrix of it in ghost clipping.  No layer
has a bias; the trainable parameters are the four projection weights and the
two RMSNorm weights (4 d^2 + 3 d F + 2 d of them).

``BlockLM`` wraps one block between a frozen token embedding and a frozen
output head (the clipped parameters are the block's) and returns logits.

The attention core runs in float32 (``scaled_dot_product_attention`` on
float32 q, k, v, cast back): bf16 batched products whose right operand is a
transposed view -- which attention's backward issues -- are avoided.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn


def rotary_tables(T: int, head_dim: int, base: float = 10000.0, device=None):
    """cos / sin tables [T, head_dim / 2] of the rotary embedding (float32)."""
    inv = 1.0 / (base ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32)
                          / head_dim))
    ang = torch.arange(T, device=device, dtype=torch.float32)[:, None] * inv[None, :]
    return torch.cos(ang), torch.sin(ang)


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate pairs (x[..., :h/2], x[..., h/2:]) of x [B, H, T, h] (float32 math)."""
    h2 = x.shape[-1] // 2
    xf = x.float()
    x1, x2 = xf[..., :h2], xf[..., h2:]
    out = torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)
    return out.to(x.dtype)


class LlamaBlock(nn.Module):
    def __init__(self, d: int = 2048, n_heads: int = 16, ffn: int = 8192, eps: float = 1e-5, *,
                 dtype=None, device=None):
        super().__init__()
        if d % n_heads:
            raise ValueError("d must be a multiple of n_heads")
        self.d, self.n_heads, self.ffn = d, n_heads, ffn
        kw = dict(dtype=dtype, device=device)
        self.attn_norm = nn.RMSNorm(d, eps=eps, **kw)
        self.qkv = nn.Linear(d, 3 * d, bias=False, **kw)
        self.o = nn.Linear(d, d, bias=False, **kw)
        self.mlp_norm = nn.RMSNorm(d, eps=eps, **kw)
        self.gate_up = nn.Linear(d, 2 * ffn, bias=False, **kw)
        self.down = nn.Linear(ffn, d, bias=False, **kw)
        self._rope = {}

    def _tables(self, T, device):
        key = (T, device)
        if key not in self._rope:
            self._rope[key] = rotary_tables(T, self.d // self.n_heads, device=device)
        return self._rope[key]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, T, d = x.shape
        H, hd = self.n_heads, d // self.n_heads
        qkv = self.qkv(self.attn_norm(x)).view(B, T, 3, H, hd)
        q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
        cos, sin = self._tables(T, x.device)
        q, k = apply_rotary(q, cos, sin), apply_rotary(k, cos, sin)
        att = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True)
        att = att.to(x.dtype).transpose(1, 2).reshape(B, T, d)
        x = x + self.o(att)
        gu = self.gate_up(self.mlp_norm(x))
        h = F.silu(gu[..., :self.ffn].float()).to(x.dtype) * gu[..., self.ffn:]
        return x + self.down(h)


class BlockLM(nn.Module):
    """Frozen embedding -> one ``LlamaBlock`` -> frozen head: logits [B, T, V]."""

    def __init__(self, vocab: int = 32000, d: int = 2048, n_heads: int = 16, ffn: int = 8192, *,
                 dtype=None, device=None):
        super().__init__()
        kw = dict(dtype=dtype, device=device)
        self.embed = nn.Embedding(vocab, d, **kw)
        self.block = LlamaBlock(d, n_heads, ffn, **kw)
        self.head = nn.Linear(d, vocab, bias=False, **kw)
        self.embed.weight.requires_grad_(False)
        self.head.weight.requires_grad_(False)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return self.head(self.block(self.embed(ids)))


def per_example_lm_loss(logits: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    """Mean next-token cross-entropy of each example (float32) [B]."""
    B, T, V = logits.shape
    ce = F.cross_entropy(logits.reshape(B * T, V).float(), targets.reshape(B * T),
                         reduction="none")
    return ce.view(B, T).mean(dim=1)


__all__ = ["BlockLM", "LlamaBlock", "apply_rotary", "per_example_lm_loss", "rotary_tables"]
