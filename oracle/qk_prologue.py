"""CPU oracle for the fused attention prologue (TEST INFRASTRUCTURE ONLY).

Only ``tests/`` (and the checker legs of ``bench.py`` / ``__graft_entry__.smoke()``) may
import this module.  The product op (``tinytrain_amd.kernels.qk_prologue``) never calls
it and has no CPU fallback.

What it restates (reference = XinqiWan412/tinytrain, files under /root/reference):

* ``rms_norm``        -- model.py:24-35: ``x`` to fp32, ``r = rsqrt(mean(x^2) + eps)``,
  ``(weight * x) * r`` in fp32, cast back to the input dtype.
* ``apply_rope``      -- model.py:48-56: cos/sin cast to the input dtype,
  ``x * cos + cat(-x2, x1) * sin`` in the input dtype (each product and the sum
  rounded to it, as torch evaluates bf16 tensor expressions).
* ``qk_prologue``     -- model.py:83-93: q/k norms on the [B, T, H, D] projections, the
  transpose to [B, H, T, D], RoPE on rows 0..T-1 of the tables, contiguous outputs
  (the ``.contiguous()`` of the "triton" branch, model.py:92-93).  Returns q, k, v and
  the per-row 1/rms (fp32, [B, T, H]) the HIP op saves for its backward.

How each function is pinned (tests/test_qk_prologue_host.py):

* ``rms_norm`` vs ``torch.nn.functional.rms_norm`` (a library routine) in fp32 and fp64,
  and its closed form on constant rows (every element c: output w * sign(c) /
  sqrt(1 + eps / c^2)).
* ``apply_rope`` in fp64: position 0 is the identity (cos 1, sin 0); each pair
  (x_i, x_{i+D/2}) is rotated by the angle of column i, so the pair norms are
  preserved and rotating by angle a then b equals rotating by a + b; one explicit
  2x2 rotation checked element by element.
* ``qk_prologue`` backward: autograd through the fp64 restatement vs
  ``torch.autograd.gradcheck`` finite differences.
* The bf16 path vs the fp64 path on the same inputs: within bf16 rounding.
"""

from __future__ import annotations

import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """model.py:30-35 (fp32 internally, result in x.dtype; fp64 stays fp64)."""
    dt = x.dtype
    xf = x.to(torch.float64 if dt == torch.float64 else torch.float32)
    r = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (weight.to(xf.dtype) * xf * r).to(dt)


def rms_rstd(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """1 / sqrt(mean(x^2) + eps) per row, fp32 (fp64 for fp64 input)."""
    xf = x.to(torch.float64 if x.dtype == torch.float64 else torch.float32)
    return torch.rsqrt(xf.pow(2).mean(dim=-1) + eps)


def rope_tables(head_dim: int, max_seq_len: int, base: float, dtype=torch.float32):
    """model.py:38-45: angles pos * base^(-2i/D), duplicated over both halves."""
    theta = base ** (-torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim)
    ang = torch.arange(max_seq_len, dtype=torch.float64)[:, None] * theta
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().to(dtype), ang.sin().to(dtype)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """model.py:48-56, in x.dtype; cos/sin [T, D] broadcast over leading dims."""
    cos, sin = cos.to(x.dtype), sin.to(x.dtype)
    x1, x2 = x.chunk(2, dim=-1)
    return x * cos + torch.cat([-x2, x1], dim=-1) * sin


def qk_prologue(q_raw: torch.Tensor, k_raw: torch.Tensor, v_raw: torch.Tensor,
                wq: torch.Tensor, wk: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                eps: float = 1e-6):
    """model.py:83-93 on [B, T, H, D] inputs -> (q, k, v [B, H, T, D] contiguous,
    rstd_q [B, T, Hq], rstd_k [B, T, Hkv])."""
    T = q_raw.shape[1]
    q = rms_norm(q_raw, wq, eps).transpose(1, 2)
    k = rms_norm(k_raw, wk, eps).transpose(1, 2)
    v = v_raw.transpose(1, 2)
    c, s = cos[:T], sin[:T]
    q, k = apply_rope(q, c, s), apply_rope(k, c, s)
    return (q.contiguous(), k.contiguous(), v.contiguous(), rms_rstd(q_raw, eps),
            rms_rstd(k_raw, eps))
