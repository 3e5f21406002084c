"""KV-cache decode attention backed by libttfa.so (inference; no backward).

``flash_attn_decode(q, k_cache, v_cache, cache_seqlens)``: q [B, Hq, Tq, D] holds the Tq
newest query rows of every sequence, whose K/V are already written at positions
cache_seqlens[b] - Tq .. cache_seqlens[b] - 1 of the [B, Hkv, max_seqlen, D] caches.
Row i attends causally to cache keys 0 .. cache_seqlens[b] - Tq + i, as the last Tq rows
of the reference's causal attention would (model.py:94-98).  Returns (o [B, Hq, Tq, D]
bf16, lse [B, Hq, Tq] fp32).  The reference regenerates the whole prefix per token
(generate.py:7-20); a KV cache is on its roadmap (README.md:158).

Supported: bf16, D in {64, 128}, Hq % Hkv == 0, (Hq / Hkv) * Tq <= 32, cache_seqlens an
int32 device tensor [B] (values clamped to 0 .. max_seqlen).
"""

from __future__ import annotations

import math

import torch

from .. import _lib
from .flash_attn import FlashAttnInputError

__all__ = ["flash_attn_decode"]


def _check(q, k_cache, v_cache, cache_seqlens):
    if q.dim() != 4 or k_cache.dim() != 4 or v_cache.dim() != 4:
        raise FlashAttnInputError("q [B, Hq, Tq, D] and caches [B, Hkv, L, D] must be 4-D")
    B, Hq, Tq, D = q.shape
    if k_cache.shape != v_cache.shape or k_cache.shape[0] != B or k_cache.shape[3] != D:
        raise FlashAttnInputError(
            f"caches must be [B, Hkv, L, D] matching q {tuple(q.shape)}; got {tuple(k_cache.shape)}")
    Hkv, L = k_cache.shape[1], k_cache.shape[2]
    if Hkv < 1 or Hq % Hkv:
        raise FlashAttnInputError(f"Hq={Hq} must be a multiple of Hkv={Hkv}")
    if D not in (64, 128):
        raise FlashAttnInputError(f"head dim D={D} is not supported (64 or 128)")
    if (Hq // Hkv) * Tq > 32:
        raise FlashAttnInputError(f"(Hq / Hkv) * Tq = {(Hq // Hkv) * Tq} exceeds 32 query rows")
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        if t.dtype != torch.bfloat16:
            raise FlashAttnInputError(f"{name} must be bfloat16")
        if not t.is_contiguous():
            raise FlashAttnInputError(f"{name} must be contiguous")
    if cache_seqlens.shape != (B,) or cache_seqlens.dtype != torch.int32:
        raise FlashAttnInputError("cache_seqlens must be an int32 tensor [B]")
    for t in (q, k_cache, v_cache, cache_seqlens):
        if t.device.type != "cuda" or t.device != q.device:
            raise FlashAttnInputError("all tensors must be on one ROCm GPU device")
    return B, Hq, Hkv, Tq, L, D


@torch.library.custom_op("tinytrain::flash_attn_decode", mutates_args=())
def flash_attn_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      cache_seqlens: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    B, Hq, Hkv, Tq, L, D = _check(q, k_cache, v_cache, cache_seqlens)
    lib = _lib.load()
    nbytes = lib.ttfa_decode_workspace_bytes(B, Hq, Hkv, Tq, L, D)
    if nbytes < 0:
        _lib.check(_lib.E_SEQ)
    ws = torch.empty((nbytes // 4 + 4,), device=q.device, dtype=torch.float32)
    o = torch.empty_like(q)
    lse = torch.empty((B, Hq, Tq), device=q.device, dtype=torch.float32)
    seqlens = cache_seqlens.contiguous()  # held until the launch is enqueued
    with torch.cuda.device(q.device):
        _lib.check(lib.ttfa_decode_fwd(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                       seqlens.data_ptr(), o.data_ptr(),
                                       lse.data_ptr(), ws.data_ptr(), B, Hq, Hkv, Tq, L, D,
                                       _lib.TTFA_BF16, 1.0 / math.sqrt(D),
                                       torch.cuda.current_stream(q.device).cuda_stream))
    return o, lse


@flash_attn_decode.register_fake
def _(q, k_cache, v_cache, cache_seqlens):
    B, Hq, Tq, D = q.shape
    return torch.empty_like(q), q.new_empty((B, Hq, Tq), dtype=torch.float32)
