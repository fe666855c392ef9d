"""LoRA adapters and a LoRA-adapted Llama-style block.

``LoRALinear`` is a frozen linear layer plus a rank-``r`` update,
``y = base(x) + (alpha / r) * lora_B(lora_A(x))`` (Hu et al., "LoRA: Low-Rank
Adaptation of Large Language Models"), with the adapters as bias-free linear
layers in the PEFT layout: ``lora_A.weight`` [r, din], ``lora_B.weight``
[dout, r].  The reference's fused kernels keep the transposes
(``A`` [din, r], ``B`` [r, dout]; packages/opake-patches/src/opake/api/patches/
kernels/lora.py:1285-1300); the per-example gradients are the same numbers.

Only the adapters are trainable, and each has a side of width r, so ghost
clipping forms their per-example gradients directly (``dpc_per_example_grads``:
2 T din r FLOP per example instead of the Gram norm's T^2 (din + r)).

``LoRABlock`` is the 8B-shaped block of the LoRA configuration: pre-norm
attention with grouped-query heads (separate q / k / v / o projections) and a
SwiGLU FFN (gate / up / down), every projection a ``LoRALinear``; the norms
and base weights are frozen.  Its attention core runs in float32.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import nn

from opake_amd.transformer import apply_rotary, rotary_tables


class LoRALinear(nn.Module):
    def __init__(self, din: int, dout: int, r: int = 16, alpha: float = 32.0, *, bias=False,
                 dtype=None, device=None):
        super().__init__()
        kw = dict(dtype=dtype, device=device)
        self.base = nn.Linear(din, dout, bias=bias, **kw)
        self.base.requires_grad_(False)
        self.lora_A = nn.Linear(din, r, bias=False, **kw)
        self.lora_B = nn.Linear(r, dout, bias=False, **kw)
        self.scaling = alpha / r
        with torch.no_grad():
            nn.init.kaiming_uniform_(self.lora_A.weight, a=math.sqrt(5))
            nn.init.zeros_(self.lora_B.weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.base(x) + self.lora_B(self.lora_A(x)) * self.scaling


class LoRABlock(nn.Module):
    def __init__(self, d: int = 4096, n_heads: int = 32, n_kv_heads: int = 8,
                 ffn: int = 14336, r: int = 16, alpha: float = 32.0, eps: float = 1e-5, *,
                 dtype=None, device=None):
        super().__init__()
        if d % n_heads or n_heads % n_kv_heads:
            raise ValueError("d must divide into n_heads, n_heads into n_kv_heads")
        self.d, self.n_heads, self.n_kv, self.ffn = d, n_heads, n_kv_heads, ffn
        hd = d // n_heads
        kw = dict(dtype=dtype, device=device)
        lk = dict(r=r, alpha=alpha, **kw)
        self.attn_norm = nn.RMSNorm(d, eps=eps, **kw)
        self.q = LoRALinear(d, d, **lk)
        self.k = LoRALinear(d, n_kv_heads * hd, **lk)
        self.v = LoRALinear(d, n_kv_heads * hd, **lk)
        self.o = LoRALinear(d, d, **lk)
        self.mlp_norm = nn.RMSNorm(d, eps=eps, **kw)
        self.gate = LoRALinear(d, ffn, **lk)
        self.up = LoRALinear(d, ffn, **lk)
        self.down = LoRALinear(ffn, d, **lk)
        self.attn_norm.requires_grad_(False)
        self.mlp_norm.requires_grad_(False)
        self._rope = {}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, T, d = x.shape
        H, KV, hd = self.n_heads, self.n_kv, d // self.n_heads
        h = self.attn_norm(x)
        q = self.q(h).view(B, T, H, hd).transpose(1, 2)
        k = self.k(h).view(B, T, KV, hd).transpose(1, 2)
        v = self.v(h).view(B, T, KV, hd).transpose(1, 2)
        key = (T, x.device)
        if key not in self._rope:
            self._rope[key] = rotary_tables(T, hd, device=x.device)
        cos, sin = self._rope[key]
        q, k = apply_rotary(q, cos, sin), apply_rotary(k, cos, sin)
        rep = H // KV
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
        att = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True)
        x = x + self.o(att.to(x.dtype).transpose(1, 2).reshape(B, T, d))
        h = self.mlp_norm(x)
        a = F.silu(self.gate(h).float()).to(x.dtype) * self.up(h)
        return x + self.down(a)


def adapter_param_count(model: nn.Module) -> int:
    return sum(p.numel() for p in model.parameters() if p.requires_grad)


__all__ = ["LoRABlock", "LoRALinear", "adapter_param_count"]
