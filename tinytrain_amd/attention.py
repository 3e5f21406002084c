"""The attention switch of the reference's model, with the HIP kernels as ``"hip"``.

Mirrors model.py:59-102 (``Attention``) and the ``attn_impl`` validation of
pretrain.py:226-231.  ``attn_impl``:

* ``"sdpa"`` -- the eager path, model.py:94-98: optional ``repeat_interleave`` GQA
  expansion, then ``F.scaled_dot_product_attention(is_causal=True)``.
* ``"hip"``  -- ``flash_attn`` on contiguous q/k/v (the call model.py:92-93 makes for
  ``"triton"``), backed by libttfa.so.  With ``Attention.fused_prologue`` set, the q/k
  norms, RoPE and the layout change run as one HIP op (``qk_norm_rope``) instead of the
  eager expressions.

An unknown name raises ``ValueError`` (no silent fallback).  ``"hip"`` on tensors the
HIP ops cannot take (CPU tensors, unsupported D) raises too.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .kernels.flash_attn import flash_attn
from .kernels.qk_prologue import qk_norm_rope

ATTN_IMPLS = ("sdpa", "hip")


def validate_attn_impl(name: str) -> str:
    """pretrain.py:226-227: reject anything but a known implementation name."""
    if name not in ATTN_IMPLS:
        raise ValueError(f"attn_impl must be one of {ATTN_IMPLS}, got {name!r}")
    return name


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attn_impl: str = "sdpa",
                     enable_gqa: bool = False) -> torch.Tensor:
    """The switch at model.py:92-98 on [B, H, T, D] / [B, H_kv, T, D] tensors."""
    validate_attn_impl(attn_impl)
    if attn_impl == "hip":
        return flash_attn(q.contiguous(), k.contiguous(), v.contiguous())
    if not enable_gqa:
        g = q.shape[1] // k.shape[1]
        k = k.repeat_interleave(g, dim=1)
        v = v.repeat_interleave(g, dim=1)
    return F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=enable_gqa)


class RMSNorm(nn.Module):
    """fp32-internal RMSNorm returning the input dtype (model.py:24-35)."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        dt = x.dtype
        x = x.float()
        return (self.weight * x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)).to(dt)


def precompute_rope(head_dim: int, max_seq_len: int, base: float):
    """(cos, sin) tables [max_seq_len, head_dim] (model.py:38-45)."""
    theta = base ** (-torch.arange(0, head_dim, 2) / head_dim)
    ang = torch.arange(max_seq_len)[:, None] * theta
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos(), ang.sin()


def apply_rope(x, cos, sin):
    """Rotate-half RoPE in the input dtype (model.py:48-56)."""
    cos, sin = cos.to(x.dtype), sin.to(x.dtype)
    x1, x2 = x.chunk(2, dim=-1)
    return x * cos + torch.cat([-x2, x1], dim=-1) * sin


class Attention(nn.Module):
    """Causal GQA self-attention block with q/k RMSNorm and RoPE (model.py:59-102)."""

    def __init__(self, hidden_size: int, num_heads: int, num_kv_heads: int, head_dim: int,
                 eps: float = 1e-6):
        super().__init__()
        self.head_dim = head_dim
        self.q_proj = nn.Linear(hidden_size, num_heads * head_dim, bias=False)
        self.k_proj = nn.Linear(hidden_size, num_kv_heads * head_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, num_kv_heads * head_dim, bias=False)
        self.o_proj = nn.Linear(num_heads * head_dim, hidden_size, bias=False)
        self.q_norm = RMSNorm(head_dim, eps)
        self.k_norm = RMSNorm(head_dim, eps)
        self.enable_gqa = False
        self.attn_impl = "sdpa"
        self.fused_prologue = False  # "hip" only: q/k norm + RoPE + layout in one HIP op

    def forward(self, x, cos, sin):
        B, T, _ = x.shape
        dh = self.head_dim
        # Head counts come from the weight shapes, so head-sharded (TP) weights work.
        H, H_kv = self.q_proj.weight.shape[0] // dh, self.k_proj.weight.shape[0] // dh
        q = self.q_proj(x).view(B, T, H, dh)
        k = self.k_proj(x).view(B, T, H_kv, dh)
        v = self.v_proj(x).view(B, T, H_kv, dh)
        # The fused op takes one eps for both norms; with different eps the eager lines
        # below run instead (the reference builds both from config.rms_norm_eps, model.py:70-71).
        if self.fused_prologue and self.attn_impl == "hip" and self.q_norm.eps == self.k_norm.eps:
            # norm + RoPE + [B, H, T, D] layout in one HIP op (replaces the next 4 lines)
            q, k, v = qk_norm_rope(q, k, v, self.q_norm.weight, self.k_norm.weight, cos, sin,
                                   self.q_norm.eps)
            out = flash_attn(q, k, v)
            return self.o_proj(out.transpose(1, 2).reshape(B, T, H * dh))
        q, k = self.q_norm(q), self.k_norm(k)
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        cos, sin = cos[:T], sin[:T]
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        out = causal_attention(q, k, v, self.attn_impl, self.enable_gqa)
        return self.o_proj(out.transpose(1, 2).reshape(B, T, H * dh))
