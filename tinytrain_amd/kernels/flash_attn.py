"""Causal GQA FlashAttention ops backed by the gfx950 HIP library (libttfa.so).

Drop-in for the reference's ``kernels/flash_attn.py`` (XinqiWan412/tinytrain): same
op names, schemas, fake implementations, autograd registration and Python entry
points (``_forward``, ``_backward``, ``flash_attn``, ``flash_attn_fwd``,
``flash_attn_bwd``; kernels/flash_attn.py:220-327), so ``model.py``'s attention
switch and ``torch.compile(fullgraph=True)`` see the same opaque nodes.

Contract (kernels/flash_attn.py:220-277):
  q [B, Hq, T, D], k/v [B, Hkv, T, D], contiguous, same dtype (bf16 or fp32), same
  ROCm device; D in {64, 128}; Hq % Hkv == 0; causal; scale 1/sqrt(D).
  ``_forward`` returns (o [B, Hq, T, D], M [B, Hq, T] fp32) with M = logsumexp of the
  scaled scores in natural-log units.  ``_backward`` returns (dq, dk, dv) in the input
  shapes.  Outputs are fresh tensors from torch's caching allocator; inputs are never
  written.  Launches are asynchronous on the current stream.

Errors: non-contiguous inputs raise ``FlashAttnInputError`` (a subclass of both
``ValueError`` and ``AssertionError``; the reference asserts contiguity at :221-223),
as do wrong ranks, shapes, dtypes, devices, D or group sizes (the reference does not
check these).  CPU tensors are rejected: there is no CPU implementation of the ops.
"""

from __future__ import annotations

import math

import torch

from .. import _lib

__all__ = ["_forward", "_backward", "flash_attn", "flash_attn_fwd", "flash_attn_bwd",
           "flash_attn_varlen", "flash_attn_varlen_fwd", "flash_attn_varlen_bwd",
           "FlashAttnInputError"]

_DTYPES = {torch.bfloat16: _lib.TTFA_BF16, torch.float32: _lib.TTFA_F32}


class FlashAttnInputError(ValueError, AssertionError):
    """Inputs outside the op contract."""


def _check_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> tuple:
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dim() != 4:
            raise FlashAttnInputError(f"{name} must be 4-D [B, H, T, D], got shape {tuple(t.shape)}")
        if not t.is_contiguous():
            raise FlashAttnInputError(f"{name} must be contiguous")
    B, Hq, T, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[2:] != (T, D):
        raise FlashAttnInputError(
            f"k/v must be [B, Hkv, T, D] matching q {tuple(q.shape)}; got k {tuple(k.shape)}, "
            f"v {tuple(v.shape)}")
    Hkv = k.shape[1]
    if Hkv < 1 or Hq % Hkv != 0:
        raise FlashAttnInputError(f"Hq={Hq} must be a multiple of Hkv={Hkv}")
    if D not in (64, 128):
        raise FlashAttnInputError(f"head dim D={D} is not supported (64 or 128)")
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise FlashAttnInputError(
            f"q/k/v must share dtype bfloat16 or float32; got {q.dtype}, {k.dtype}, {v.dtype}")
    if q.device.type != "cuda" or k.device != q.device or v.device != q.device:
        raise FlashAttnInputError(
            f"q/k/v must be on one ROCm GPU device; got {q.device}, {k.device}, {v.device} "
            "(the HIP library is the only implementation)")
    return B, Hq, Hkv, T, D


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _forward(q, k, v):
    """Forward launcher (kernels/flash_attn.py:220-243): returns (o, M)."""
    B, H, H_kv, T, D = _check_qkv(q, k, v)
    lib = _lib.load()
    o = torch.empty_like(q)
    M = torch.empty((B, H, T), device=q.device, dtype=torch.float32)
    with torch.cuda.device(q.device):
        _lib.check(lib.ttfa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                M.data_ptr(), B, H, H_kv, T, D, _DTYPES[q.dtype],
                                1.0 / math.sqrt(D), _stream_ptr(q.device)))
    return o, M


def _backward(q, k, v, o, do, M):
    """Backward launcher (kernels/flash_attn.py:246-277): returns (dq, dk, dv)."""
    B, H, H_kv, T, D = _check_qkv(q, k, v)
    do = do.contiguous()
    o = o.contiguous()
    for name, t in (("o", o), ("do", do)):
        if t.shape != q.shape or t.dtype != q.dtype or t.device != q.device:
            raise FlashAttnInputError(f"{name} must match q in shape, dtype and device")
    if M.shape != (B, H, T) or M.dtype != torch.float32 or M.device != q.device:
        raise FlashAttnInputError("M must be the forward's fp32 [B, Hq, T] logsumexp")
    M = M.contiguous()
    lib = _lib.load()
    delta = torch.empty((B * H, T), device=q.device, dtype=torch.float32)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    with torch.cuda.device(q.device):
        _lib.check(lib.ttfa_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                do.data_ptr(), M.data_ptr(), delta.data_ptr(), dq.data_ptr(),
                                dk.data_ptr(), dv.data_ptr(), B, H, H_kv, T, D,
                                _DTYPES[q.dtype], 1.0 / math.sqrt(D), _stream_ptr(q.device)))
    return dq, dk, dv


# ---------------------------------------------------------------------------------------
# custom op registration: torch.compile sees each op as one opaque node
# (kernels/flash_attn.py:284-321)
# ---------------------------------------------------------------------------------------

@torch.library.custom_op("tinytrain::flash_attn_fwd", mutates_args=())
def flash_attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor
                   ) -> tuple[torch.Tensor, torch.Tensor]:
    return _forward(q, k, v)


@flash_attn_fwd.register_fake
def _(q, k, v):
    B, H, T, D = q.shape
    return torch.empty_like(q), q.new_empty((B, H, T), dtype=torch.float32)


@torch.library.custom_op("tinytrain::flash_attn_bwd", mutates_args=())
def flash_attn_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   o: torch.Tensor, do: torch.Tensor, M: torch.Tensor
                   ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _backward(q, k, v, o, do, M)


@flash_attn_bwd.register_fake
def _(q, k, v, o, do, M):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _setup_context(ctx, inputs, output):
    q, k, v = inputs
    o, M = output
    ctx.save_for_backward(q, k, v, o, M)


def _backward_fn(ctx, do, dM):
    # M only feeds the backward; its gradient is ignored (kernels/flash_attn.py:315-318).
    q, k, v, o, M = ctx.saved_tensors
    return flash_attn_bwd(q, k, v, o, do, M)


flash_attn_fwd.register_autograd(_backward_fn, setup_context=_setup_context)


def flash_attn(q, k, v):
    """Causal attention on contiguous [B, H, T, D] / [B, H_kv, T, D]; returns o."""
    o, _ = flash_attn_fwd(q, k, v)
    return o


# ---------------------------------------------------------------------------------------
# packed variable-length sequences (cu_seqlens): the varlen item of the reference's
# roadmap (README.md:158), on the same kernels as the batched ops
# ---------------------------------------------------------------------------------------

def _check_varlen(q, k, v, cu_seqlens, max_seqlen):
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dim() != 3:
            raise FlashAttnInputError(f"{name} must be 3-D [H, total, D], got shape {tuple(t.shape)}")
        if not t.is_contiguous():
            raise FlashAttnInputError(f"{name} must be contiguous")
    Hq, total, D = q.shape
    if k.shape != v.shape or k.shape[1:] != (total, D):
        raise FlashAttnInputError(
            f"k/v must be [Hkv, total, D] matching q {tuple(q.shape)}; got {tuple(k.shape)}")
    Hkv = k.shape[0]
    if Hkv < 1 or Hq % Hkv:
        raise FlashAttnInputError(f"Hq={Hq} must be a multiple of Hkv={Hkv}")
    if D not in (64, 128):
        raise FlashAttnInputError(f"head dim D={D} is not supported (64 or 128)")
    if q.dtype != torch.bfloat16 or k.dtype != q.dtype or v.dtype != q.dtype:
        raise FlashAttnInputError("varlen attention takes bfloat16 q/k/v")
    if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2 or cu_seqlens.dtype != torch.int32:
        raise FlashAttnInputError("cu_seqlens must be a 1-D int32 tensor of n_seq + 1 offsets")
    if not cu_seqlens.is_contiguous():
        raise FlashAttnInputError("cu_seqlens must be contiguous")
    if int(max_seqlen) < 1 or total < 1:
        raise FlashAttnInputError("max_seqlen and total must be >= 1")
    for t in (q, k, v, cu_seqlens):
        if t.device.type != "cuda" or t.device != q.device:
            raise FlashAttnInputError("q/k/v/cu_seqlens must be on one ROCm GPU device")
    return Hq, Hkv, total, D, cu_seqlens.numel() - 1


def _varlen_forward(q, k, v, cu_seqlens, max_seqlen):
    Hq, Hkv, total, D, n_seq = _check_varlen(q, k, v, cu_seqlens, max_seqlen)
    lib = _lib.load()
    o = torch.empty_like(q)
    M = torch.empty((Hq, total), device=q.device, dtype=torch.float32)
    with torch.cuda.device(q.device):
        _lib.check(lib.ttfa_varlen_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                       M.data_ptr(), cu_seqlens.data_ptr(), n_seq, total,
                                       int(max_seqlen), Hq, Hkv, D, _lib.TTFA_BF16,
                                       1.0 / math.sqrt(D), _stream_ptr(q.device)))
    return o, M


def _varlen_backward(q, k, v, o, do, M, cu_seqlens, max_seqlen):
    Hq, Hkv, total, D, n_seq = _check_varlen(q, k, v, cu_seqlens, max_seqlen)
    do, o, M = do.contiguous(), o.contiguous(), M.contiguous()
    if do.shape != q.shape or o.shape != q.shape or do.dtype != q.dtype or o.dtype != q.dtype:
        raise FlashAttnInputError("o/do must match q in shape and dtype")
    if M.shape != (Hq, total) or M.dtype != torch.float32:
        raise FlashAttnInputError("M must be the forward's fp32 [Hq, total] logsumexp")
    lib = _lib.load()
    delta = torch.empty((Hq, total), device=q.device, dtype=torch.float32)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    with torch.cuda.device(q.device):
        _lib.check(lib.ttfa_varlen_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                       do.data_ptr(), M.data_ptr(), delta.data_ptr(), dq.data_ptr(),
                                       dk.data_ptr(), dv.data_ptr(), cu_seqlens.data_ptr(), n_seq,
                                       total, int(max_seqlen), Hq, Hkv, D, _lib.TTFA_BF16,
                                       1.0 / math.sqrt(D), _stream_ptr(q.device)))
    return dq, dk, dv


@torch.library.custom_op("tinytrain::flash_attn_varlen_fwd", mutates_args=())
def flash_attn_varlen_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          cu_seqlens: torch.Tensor, max_seqlen: int
                          ) -> tuple[torch.Tensor, torch.Tensor]:
    return _varlen_forward(q, k, v, cu_seqlens, max_seqlen)


@flash_attn_varlen_fwd.register_fake
def _(q, k, v, cu_seqlens, max_seqlen):
    H, total, D = q.shape
    return torch.empty_like(q), q.new_empty((H, total), dtype=torch.float32)


@torch.library.custom_op("tinytrain::flash_attn_varlen_bwd", mutates_args=())
def flash_attn_varlen_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                          do: torch.Tensor, M: torch.Tensor, cu_seqlens: torch.Tensor,
                          max_seqlen: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _varlen_backward(q, k, v, o, do, M, cu_seqlens, max_seqlen)


@flash_attn_varlen_bwd.register_fake
def _(q, k, v, o, do, M, cu_seqlens, max_seqlen):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _varlen_setup_context(ctx, inputs, output):
    q, k, v, cu_seqlens, max_seqlen = inputs
    o, M = output
    ctx.save_for_backward(q, k, v, o, M, cu_seqlens)
    ctx.max_seqlen = max_seqlen


def _varlen_backward_fn(ctx, do, dM):
    q, k, v, o, M, cu_seqlens = ctx.saved_tensors
    dq, dk, dv = flash_attn_varlen_bwd(q, k, v, o, do, M, cu_seqlens, ctx.max_seqlen)
    return dq, dk, dv, None, None


flash_attn_varlen_fwd.register_autograd(_varlen_backward_fn, setup_context=_varlen_setup_context)


def flash_attn_varlen(q, k, v, cu_seqlens, max_seqlen):
    """Causal attention over packed sequences: q [Hq, total, D], k/v [Hkv, total, D] bf16,
    cu_seqlens int32 [n_seq + 1] (device), every sequence attending only within itself;
    returns o [Hq, total, D]."""
    o, _ = flash_attn_varlen_fwd(q, k, v, cu_seqlens, int(max_seqlen))
    return o
