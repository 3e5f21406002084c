"""Decoder-only language model shaped like the reference's, for the whole-model check of
the attention switch: logits parity between ``attn_impl`` values and the training-step
throughput benchmark (``python bench.py --model``).

Structure and defaults follow the reference's model.py: ``ModelConfig`` (:9-21, the
112M pretrain shape: hidden 768, 12 layers, 8 query / 2 KV heads of 128, SwiGLU 2304,
T <= 512, RoPE base 1e6, tied embeddings), pre-norm blocks (:128-139), final RMSNorm and
a tied LM head with mean cross-entropy (:143-212), normal(0, 0.02) init (:183-186).
Attention, RMSNorm and RoPE come from ``tinytrain_amd.attention``.  Chunked
cross-entropy and activation checkpointing (reference training options) are not part of
this benchmark model.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch.nn as nn
import torch.nn.functional as F

from .attention import Attention, RMSNorm, precompute_rope, validate_attn_impl


@dataclass
class ModelConfig:
    vocab_size: int = 32768
    hidden_size: int = 768
    num_hidden_layers: int = 12
    num_attention_heads: int = 8
    num_key_value_heads: int = 2
    head_dim: int = 128
    intermediate_size: int = 3 * 768
    max_seq_len: int = 512
    rope_theta: float = 1e6
    rms_norm_eps: float = 1e-6
    tie_word_embeddings: bool = True

    def params(self) -> int:
        """Trainable parameters (embedding counted once when tied)."""
        h, dh = self.hidden_size, self.head_dim
        attn = h * dh * (self.num_attention_heads * 2 + self.num_key_value_heads * 2) + 2 * dh
        mlp = 3 * h * self.intermediate_size
        per_layer = attn + mlp + 2 * h
        head = 0 if self.tie_word_embeddings else self.vocab_size * h
        return self.vocab_size * h + self.num_hidden_layers * per_layer + h + head

    def train_flop_per_token(self, T: int) -> float:
        """Training FLOPs per token: 6 x the weights used in matmuls (projections, MLP and
        the LM head; not the embedding lookup) plus causal attention, whose forward costs
        2 * T * dh * Hq per token and layer (QK^T and PV over T/2 keys on average) and
        whose forward + backward costs three times that."""
        h, dh = self.hidden_size, self.head_dim
        per_layer = h * dh * 2 * (self.num_attention_heads + self.num_key_value_heads) \
            + 3 * h * self.intermediate_size
        matmul_weights = self.num_hidden_layers * per_layer + self.vocab_size * h
        attn = 3 * 2 * T * dh * self.num_attention_heads * self.num_hidden_layers
        return 6.0 * matmul_weights + attn


class MLP(nn.Module):
    """SwiGLU feed-forward (model.py:111-125)."""

    def __init__(self, c: ModelConfig):
        super().__init__()
        self.gate_proj = nn.Linear(c.hidden_size, c.intermediate_size, bias=False)
        self.up_proj = nn.Linear(c.hidden_size, c.intermediate_size, bias=False)
        self.down_proj = nn.Linear(c.intermediate_size, c.hidden_size, bias=False)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class Block(nn.Module):
    """Pre-norm residual block: x + attn(norm(x)), then + mlp(norm(.)) (model.py:128-139)."""

    def __init__(self, c: ModelConfig):
        super().__init__()
        self.input_layernorm = RMSNorm(c.hidden_size, c.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(c.hidden_size, c.rms_norm_eps)
        self.self_attn = Attention(c.hidden_size, c.num_attention_heads, c.num_key_value_heads,
                                   c.head_dim, c.rms_norm_eps)
        self.mlp = MLP(c)

    def forward(self, x, cos, sin):
        h = x + self.self_attn(self.input_layernorm(x), cos, sin)
        return h + self.mlp(self.post_attention_layernorm(h))


class ModelForCausalLM(nn.Module):
    """Embedding, blocks, final norm, tied LM head; returns (logits, loss)."""

    def __init__(self, c: ModelConfig):
        super().__init__()
        self.config = c
        self.embed_tokens = nn.Embedding(c.vocab_size, c.hidden_size)
        self.layers = nn.ModuleList(Block(c) for _ in range(c.num_hidden_layers))
        self.norm = RMSNorm(c.hidden_size, c.rms_norm_eps)
        self.lm_head = nn.Linear(c.hidden_size, c.vocab_size, bias=False)
        cos, sin = precompute_rope(c.head_dim, c.max_seq_len, c.rope_theta)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)
        for mod in self.modules():
            if isinstance(mod, (nn.Linear, nn.Embedding)):
                nn.init.normal_(mod.weight, mean=0.0, std=0.02)
        if c.tie_word_embeddings:
            self.lm_head.weight = self.embed_tokens.weight

    def set_attn_impl(self, attn_impl: str, fused_prologue: bool = False,
                      enable_gqa: bool = False) -> None:
        """Select the attention path of every block (the reference sets
        ``Attention.attn_impl`` per module, tests/test_flash_attn.py:128-130)."""
        validate_attn_impl(attn_impl)
        for mod in self.modules():
            if isinstance(mod, Attention):
                mod.attn_impl = attn_impl
                mod.fused_prologue = fused_prologue
                mod.enable_gqa = enable_gqa

    def forward(self, input_ids, targets=None):
        B, T = input_ids.shape
        if T > self.config.max_seq_len:
            raise ValueError(f"T={T} exceeds max_seq_len={self.config.max_seq_len}")
        x = self.embed_tokens(input_ids)
        cos, sin = self.cos[:T], self.sin[:T]
        for blk in self.layers:
            x = blk(x, cos, sin)
        logits = self.lm_head(self.norm(x))
        loss = None
        if targets is not None:
            loss = F.cross_entropy(logits.view(B * T, -1), targets.view(B * T))
        return logits, loss
