"""Fused attention prologue ops: q/k RMSNorm + RoPE + layout change, backed by libttfa.so.

Replaces, in one HIP pass per direction, the steps the reference's Attention.forward
runs between its projections and the attention call (model.py:83-93):

    q = q_norm(q_proj(x).view(B, T, H, dh))          # RMSNorm, model.py:24-35
    k = k_norm(k_proj(x).view(B, T, H_kv, dh))
    q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)   # model.py:48-56
    flash_attn(q.contiguous(), k.contiguous(), v.contiguous())

``qk_norm_rope(q_raw, k_raw, v_raw, wq, wk, cos, sin, eps)`` takes the projections
viewed as [B, T, H, D] (contiguous) and returns contiguous q [B, H, T, D] and k, v
[B, H_kv, T, D], ready for ``flash_attn``.  bf16 only (the training dtype under
autocast); the norm weights are the fp32 parameters, cos/sin the fp32 RoPE tables
(rounded to bf16 inside, as apply_rope does).  Gradients flow to q_raw, k_raw, v_raw and
both norm weights; cos/sin get none (the reference's tables are buffers).

The forward repeats the reference's roundings (fp32 norm rounded to bf16, then bf16
products and sum for RoPE), so it matches the eager expressions to within the fp32
summation order of mean(x^2).  The backward evaluates the exact derivative of the same
expressions in fp32 and rounds once.
"""

from __future__ import annotations

import torch

from .. import _lib

__all__ = ["qk_norm_rope", "qk_norm_rope_fwd", "qk_norm_rope_bwd", "QKPrologueInputError"]


class QKPrologueInputError(ValueError):
    """Inputs outside the op contract."""


def _check(q_raw, k_raw, v_raw, wq, wk, cos, sin):
    if q_raw.dim() != 4 or k_raw.dim() != 4 or v_raw.dim() != 4:
        raise QKPrologueInputError("q_raw, k_raw, v_raw must be 4-D [B, T, H, D]")
    B, T, Hq, D = q_raw.shape
    if k_raw.shape != v_raw.shape or k_raw.shape[0] != B or k_raw.shape[1] != T or k_raw.shape[3] != D:
        raise QKPrologueInputError(
            f"k_raw/v_raw must be [B, T, H_kv, D] matching q_raw {tuple(q_raw.shape)}")
    Hkv = k_raw.shape[2]
    if Hkv < 1 or Hq % Hkv:
        raise QKPrologueInputError(f"Hq={Hq} must be a multiple of Hkv={Hkv}")
    if D not in (64, 128):
        raise QKPrologueInputError(f"head dim D={D} is not supported (64 or 128)")
    for name, t in (("q_norm weight", wq), ("k_norm weight", wk)):
        if t.shape != (D,):
            raise QKPrologueInputError(f"{name} must be [D] = [{D}], got {tuple(t.shape)}")
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[0] < T or cos.shape[1] != D:
        raise QKPrologueInputError(f"cos/sin must be [>= T, D] tables, got {tuple(cos.shape)}")
    for name, t in (("q_raw", q_raw), ("k_raw", k_raw), ("v_raw", v_raw)):
        if t.dtype != torch.bfloat16:
            raise QKPrologueInputError(f"{name} must be bfloat16, got {t.dtype}")
        if not t.is_contiguous():
            raise QKPrologueInputError(f"{name} must be contiguous")
    for t in (q_raw, k_raw, v_raw, wq, wk):
        if t.device.type != "cuda" or t.device != q_raw.device:
            raise QKPrologueInputError(
                "inputs and norm weights must be on one ROCm GPU device (the HIP library is "
                "the only implementation)")
    return B, T, Hq, Hkv, D


def _tables(cos, sin, T, device):
    """Rows 0..T-1 of the RoPE tables in bf16 (apply_rope's cos.to(x.dtype))."""
    return (cos[:T].to(device=device, dtype=torch.bfloat16).contiguous(),
            sin[:T].to(device=device, dtype=torch.bfloat16).contiguous())


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _fwd(q_raw, k_raw, v_raw, wq, wk, cos, sin, eps):
    B, T, Hq, Hkv, D = _check(q_raw, k_raw, v_raw, wq, wk, cos, sin)
    dev = q_raw.device
    cb, sb = _tables(cos, sin, T, dev)
    wq32, wk32 = wq.float().contiguous(), wk.float().contiguous()
    q = torch.empty((B, Hq, T, D), device=dev, dtype=torch.bfloat16)
    k = torch.empty((B, Hkv, T, D), device=dev, dtype=torch.bfloat16)
    v = torch.empty((B, Hkv, T, D), device=dev, dtype=torch.bfloat16)
    rq = torch.empty((B, T, Hq), device=dev, dtype=torch.float32)
    rk = torch.empty((B, T, Hkv), device=dev, dtype=torch.float32)
    lib = _lib.load()
    with torch.cuda.device(dev):
        _lib.check(lib.ttfa_qk_prologue_fwd(
            q_raw.data_ptr(), k_raw.data_ptr(), v_raw.data_ptr(), wq32.data_ptr(),
            wk32.data_ptr(), cb.data_ptr(), sb.data_ptr(), q.data_ptr(), k.data_ptr(),
            v.data_ptr(), rq.data_ptr(), rk.data_ptr(), B, T, Hq, Hkv, D, float(eps),
            _stream(dev)))
    return q, k, v, rq, rk


def _bwd(dq, dk, dv, q_raw, k_raw, wq, wk, cos, sin, rq, rk):
    B, T, Hq, D = q_raw.shape
    Hkv = k_raw.shape[2]
    dev = q_raw.device
    cb, sb = _tables(cos, sin, T, dev)
    wq32, wk32 = wq.float().contiguous(), wk.float().contiguous()
    dq, dk, dv = (t.to(torch.bfloat16).contiguous() for t in (dq, dk, dv))
    dq_raw = torch.empty_like(q_raw)
    dk_raw = torch.empty_like(k_raw)
    dv_raw = torch.empty_like(k_raw)
    dwq = torch.empty((D,), device=dev, dtype=torch.float32)
    dwk = torch.empty((D,), device=dev, dtype=torch.float32)
    lib = _lib.load()
    nbytes = lib.ttfa_qk_prologue_workspace_bytes(B, T, Hq, Hkv, D)
    if nbytes < 0:
        _lib.check(_lib.E_SEQ)
    ws = torch.empty((max(nbytes // 4, 4),), device=dev, dtype=torch.float32)
    with torch.cuda.device(dev):
        _lib.check(lib.ttfa_qk_prologue_bwd(
            dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), q_raw.data_ptr(), k_raw.data_ptr(),
            wq32.data_ptr(), wk32.data_ptr(), cb.data_ptr(), sb.data_ptr(), rq.data_ptr(),
            rk.data_ptr(), dq_raw.data_ptr(), dk_raw.data_ptr(), dv_raw.data_ptr(),
            dwq.data_ptr(), dwk.data_ptr(), ws.data_ptr(), B, T, Hq, Hkv, D, _stream(dev)))
    return dq_raw, dk_raw, dv_raw, dwq.to(wq.dtype), dwk.to(wk.dtype)


@torch.library.custom_op("tinytrain::qk_norm_rope_fwd", mutates_args=())
def qk_norm_rope_fwd(q_raw: torch.Tensor, k_raw: torch.Tensor, v_raw: torch.Tensor,
                     wq: torch.Tensor, wk: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                     eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                          torch.Tensor]:
    return _fwd(q_raw, k_raw, v_raw, wq, wk, cos, sin, eps)


@qk_norm_rope_fwd.register_fake
def _(q_raw, k_raw, v_raw, wq, wk, cos, sin, eps):
    B, T, Hq, D = q_raw.shape
    Hkv = k_raw.shape[2]
    return (q_raw.new_empty((B, Hq, T, D)), k_raw.new_empty((B, Hkv, T, D)),
            k_raw.new_empty((B, Hkv, T, D)), q_raw.new_empty((B, T, Hq), dtype=torch.float32),
            k_raw.new_empty((B, T, Hkv), dtype=torch.float32))


@torch.library.custom_op("tinytrain::qk_norm_rope_bwd", mutates_args=())
def qk_norm_rope_bwd(dq: torch.Tensor, dk: torch.Tensor, dv: torch.Tensor, q_raw: torch.Tensor,
                     k_raw: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, cos: torch.Tensor,
                     sin: torch.Tensor, rq: torch.Tensor, rk: torch.Tensor
                     ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                torch.Tensor]:
    return _bwd(dq, dk, dv, q_raw, k_raw, wq, wk, cos, sin, rq, rk)


@qk_norm_rope_bwd.register_fake
def _(dq, dk, dv, q_raw, k_raw, wq, wk, cos, sin, rq, rk):
    return (torch.empty_like(q_raw), torch.empty_like(k_raw), torch.empty_like(k_raw),
            torch.empty_like(wq), torch.empty_like(wk))


def _setup_context(ctx, inputs, output):
    q_raw, k_raw, v_raw, wq, wk, cos, sin, eps = inputs
    _, _, _, rq, rk = output
    ctx.save_for_backward(q_raw, k_raw, wq, wk, cos, sin, rq, rk)


def _backward_fn(ctx, dq, dk, dv, drq, drk):
    q_raw, k_raw, wq, wk, cos, sin, rq, rk = ctx.saved_tensors
    dq_raw, dk_raw, dv_raw, dwq, dwk = qk_norm_rope_bwd(dq, dk, dv, q_raw, k_raw, wq, wk, cos,
                                                        sin, rq, rk)
    return dq_raw, dk_raw, dv_raw, dwq, dwk, None, None, None


qk_norm_rope_fwd.register_autograd(_backward_fn, setup_context=_setup_context)


def qk_norm_rope(q_raw, k_raw, v_raw, wq, wk, cos, sin, eps: float = 1e-6):
    """(q, k, v) for ``flash_attn`` from the [B, T, H, D] projections; see module doc."""
    q, k, v, _, _ = qk_norm_rope_fwd(q_raw, k_raw, v_raw, wq, wk, cos, sin, float(eps))
    return q, k, v
