"""CPU oracle for causal GQA attention (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this module, and only as the checker.  The product path
(``tinytrain_amd``) never calls it and has no CPU fallback.

What it restates (reference = XinqiWan412/tinytrain, files under /root/reference):

* ``eager_attention``      -- model.py:94-98, the ``attn_impl == "sdpa"`` branch:
  ``repeat_interleave`` GQA expansion of k/v, then
  ``F.scaled_dot_product_attention(q, k, v, is_causal=True)``.  This is the parity
  contract; the reference's own FA test compares against the same routine in fp32
  (tests/test_flash_attn.py:23-30).
* ``attention_fwd``        -- the closed form the reference kernel computes:
  ``s = q k^T * scale`` (kernels/flash_attn.py:49), causal mask (:50-53),
  ``O = softmax(s) v`` (:55-63) and ``LSE = m + ln(l)`` in natural-log units of the
  scaled scores, fp32, shape [B, Hq, T] (:67, :232).
* ``attention_delta``      -- ``Delta = rowsum(O * dO)`` (kernels/flash_attn.py:70-90).
* ``attention_bwd_rows`` / ``attention_bwd_keys`` -- the same formulas for sampled query
  rows (dQ) or keys (dK, dV) only, each from its own row or column of scores, for lengths
  where the full backward is too slow on the CPU.
* ``attention_bwd``        -- the backward formulas of kernels/flash_attn.py:93-217:
  ``P = exp(s*scale - LSE)`` (:143-145), ``dV = P^T dO`` (:147), ``dP = dO V^T`` (:149),
  ``dS = P (dP - Delta)`` (:150), ``dK = dS^T Q * scale`` (:152-154),
  ``dQ = dS K * scale`` (:213-216); dK/dV summed over the G query heads that share a
  KV head (:125-127), query head h reading KV head h // G (:24, :227).

How each function is pinned (tests/test_oracle.py):

* ``eager_attention`` vs ``attention_fwd``: two independent implementations (torch's
  SDPA library kernel vs explicit chunked matmuls in fp64) must agree.
* ``attention_fwd`` special cases fixed by the mathematics: T=1 gives O=v and
  LSE = q.k*scale; q=0 gives O_i = mean_{j<=i} v_j and LSE_i = ln(i+1);
  sum_j exp(s_ij - LSE_i) = 1; causality (changing the last key/value row changes only
  the last output row, as tests/test_model.py:49-63 checks for the module).
* ``attention_bwd`` vs autograd through ``eager_attention`` (SDPA backward), and vs
  ``torch.autograd.gradcheck`` finite differences of ``attention_fwd`` in fp64, which
  fixes every gradient formula independently of how it is written here.
* ``attention_bwd_rows`` / ``attention_bwd_keys`` vs ``attention_bwd`` on every row and key
  of small GQA inputs, and a planted missing Delta in the key form is caught.
* GQA: result equals running with k/v expanded by ``repeat_interleave``, with dK/dV
  equal to the group sum of the expanded gradients (tests/test_model.py:174-200).
* A brute-force scalar pure-Python loop on tiny inputs (``brute_force_attention``).

The reference publishes no frozen attention vectors, so these checks are the pin.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

Tensor = torch.Tensor

# Query rows per chunk in the explicit implementations (bounds the [rows, T] score
# block held at once, so T=16384 fits in a few hundred MB).
_CHUNK = 1024


def _group(q: Tensor, k: Tensor) -> int:
    Hq, Hkv = q.shape[1], k.shape[1]
    if Hq % Hkv != 0:
        raise ValueError(f"Hq={Hq} is not a multiple of Hkv={Hkv}")
    return Hq // Hkv


def eager_attention(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """model.py:94-98 restated: repeat_interleave(g) on k, v, then causal SDPA.

    Inputs are upcast to fp32 first, as tests/test_flash_attn.py:24-26 does for bf16.
    Differentiable: call ``.backward`` on the result to get the reference gradients
    (autograd sums dK/dV over the group through ``repeat_interleave``).
    """
    g = _group(q, k)
    q, k, v = q.float(), k.float(), v.float()
    k = k.repeat_interleave(g, dim=1)
    v = v.repeat_interleave(g, dim=1)
    return F.scaled_dot_product_attention(q, k, v, is_causal=True)


def eager_attention_grads(q: Tensor, k: Tensor, v: Tensor, do: Tensor
                          ) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """(O, dQ, dK, dV) in fp32 through autograd of :func:`eager_attention`."""
    qr = q.detach().float().requires_grad_()
    kr = k.detach().float().requires_grad_()
    vr = v.detach().float().requires_grad_()
    o = eager_attention(qr, kr, vr)
    o.backward(do.float())
    return o.detach(), qr.grad, kr.grad, vr.grad


def _scores_chunk(q: Tensor, k: Tensor, r0: int, r1: int, scale: float) -> Tensor:
    """Scaled, causally masked scores for query rows [r0, r1) against keys [0, r1)."""
    s = torch.matmul(q[..., r0:r1, :], k[..., :r1, :].transpose(-1, -2)) * scale
    rows = torch.arange(r0, r1, device=q.device)[:, None]
    cols = torch.arange(0, r1, device=q.device)[None, :]
    return s.masked_fill(cols > rows, float("-inf"))


def attention_fwd(q: Tensor, k: Tensor, v: Tensor, dtype: torch.dtype = torch.float64,
                  scale: Optional[float] = None) -> Tuple[Tensor, Tensor]:
    """Explicit causal GQA attention.  Returns (O [B,Hq,T,D], LSE [B,Hq,T]) in ``dtype``.

    kernels/flash_attn.py:49-67: s = q k^T * scale, causal mask, O = softmax(s) v,
    LSE = m + ln(l) (natural log of the scaled scores).
    """
    B, Hq, T, D = q.shape
    g = _group(q, k)
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    q = q.to(dtype)
    k = k.to(dtype).repeat_interleave(g, dim=1)
    v = v.to(dtype).repeat_interleave(g, dim=1)
    o = torch.empty(B, Hq, T, D, dtype=dtype)
    lse = torch.empty(B, Hq, T, dtype=dtype)
    for b in range(B):  # one sequence at a time bounds the score block's memory
        for r0 in range(0, T, _CHUNK):
            r1 = min(T, r0 + _CHUNK)
            s = _scores_chunk(q[b], k[b], r0, r1, scale)
            m = s.amax(dim=-1, keepdim=True)
            p = torch.exp(s - m)
            l = p.sum(dim=-1, keepdim=True)
            o[b, :, r0:r1, :] = torch.matmul(p, v[b, :, :r1, :]) / l
            lse[b, :, r0:r1] = (m + torch.log(l)).squeeze(-1)
    return o, lse


def attention_delta(o: Tensor, do: Tensor, dtype: torch.dtype = torch.float64) -> Tensor:
    """Delta = rowsum(O * dO) over D (kernels/flash_attn.py:85-90)."""
    return (o.to(dtype) * do.to(dtype)).sum(dim=-1)


def attention_bwd(q: Tensor, k: Tensor, v: Tensor, o: Tensor, do: Tensor, lse: Tensor,
                  dtype: torch.dtype = torch.float64, scale: Optional[float] = None
                  ) -> Tuple[Tensor, Tensor, Tensor]:
    """Explicit causal GQA attention backward.  Returns (dQ, dK, dV) in ``dtype``.

    Recomputes P from the saved LSE (kernels/flash_attn.py:143-145) and applies
    dV = P^T dO, dP = dO V^T, dS = P (dP - Delta), dQ = dS K * scale,
    dK = dS^T Q * scale, summing dK/dV over the query heads of each KV group.
    """
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    g = _group(q, k)
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    q = q.to(dtype)
    ke = k.to(dtype).repeat_interleave(g, dim=1)
    ve = v.to(dtype).repeat_interleave(g, dim=1)
    do = do.to(dtype)
    lse = lse.to(dtype)
    delta = attention_delta(o, do, dtype)
    dq = torch.zeros(B, Hq, T, D, dtype=dtype)
    dke = torch.zeros(B, Hq, T, D, dtype=dtype)
    dve = torch.zeros(B, Hq, T, D, dtype=dtype)
    for b in range(B):
        for r0 in range(0, T, _CHUNK):
            r1 = min(T, r0 + _CHUNK)
            s = _scores_chunk(q[b], ke[b], r0, r1, scale)
            p = torch.exp(s - lse[b, :, r0:r1, None])
            dorow = do[b, :, r0:r1, :]
            dve[b, :, :r1, :] += torch.matmul(p.transpose(-1, -2), dorow)
            dp = torch.matmul(dorow, ve[b, :, :r1, :].transpose(-1, -2))
            ds = p * (dp - delta[b, :, r0:r1, None])
            dq[b, :, r0:r1, :] = torch.matmul(ds, ke[b, :, :r1, :]) * scale
            dke[b, :, :r1, :] += torch.matmul(ds.transpose(-1, -2), q[b, :, r0:r1, :]) * scale
    dk = dke.view(B, Hkv, g, T, D).sum(dim=2)
    dv = dve.view(B, Hkv, g, T, D).sum(dim=2)
    return dq, dk, dv


def attention_bwd_rows(q: Tensor, k: Tensor, v: Tensor, do: Tensor, o: Tensor, lse: Tensor,
                       b: int, h: int, rows, scale: Optional[float] = None) -> Tensor:
    """dQ of the given query rows of (batch b, query head h), in fp64, from each row's own
    scores only (kernels/flash_attn.py:196-216): dQ_i = scale * sum_{j<=i} P_ij (dP_ij - Delta_i)
    K_j with P_ij = exp(s_ij - LSE_i), dP_ij = dO_i . V_j, Delta_i = O_i . dO_i.  ``o`` and
    ``lse`` are the forward's outputs for every row.  Returns [len(rows), D]."""
    D = q.shape[-1]
    g = _group(q, k)
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    out = []
    for i in rows:
        K, V = k[b, h // g, :i + 1].double(), v[b, h // g, :i + 1].double()
        dor = do[b, h, i].double()
        p = torch.exp((K @ q[b, h, i].double()) * scale - lse[b, h, i].double())
        delta = (o[b, h, i].double() * dor).sum()
        out.append(((p * (V @ dor - delta))[:, None] * K).sum(0) * scale)
    return torch.stack(out)


def attention_bwd_keys(q: Tensor, k: Tensor, v: Tensor, do: Tensor, o: Tensor, lse: Tensor,
                       b: int, hk: int, keys, scale: Optional[float] = None
                       ) -> Tuple[Tensor, Tensor]:
    """dK and dV of the given keys of (batch b, KV head hk), in fp64, from each key's own
    column of scores over the rows i >= j, summed over the KV head's query heads
    (kernels/flash_attn.py:121-159): dV_j = sum P_ij dO_i, dK_j = scale * sum P_ij
    (dP_ij - Delta_i) Q_i.  Returns ([len(keys), D], [len(keys), D])."""
    D = q.shape[-1]
    g = _group(q, k)
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    dks, dvs = [], []
    for j in keys:
        dk = torch.zeros(D, dtype=torch.float64)
        dv = torch.zeros(D, dtype=torch.float64)
        kj, vj = k[b, hk, j].double(), v[b, hk, j].double()
        for h in range(hk * g, (hk + 1) * g):
            Q, dO = q[b, h, j:].double(), do[b, h, j:].double()
            p = torch.exp((Q @ kj) * scale - lse[b, h, j:].double())
            delta = (o[b, h, j:].double() * dO).sum(-1)
            dv += (p[:, None] * dO).sum(0)
            dk += ((p * (dO @ vj - delta))[:, None] * Q).sum(0) * scale
        dks.append(dk)
        dvs.append(dv)
    return torch.stack(dks), torch.stack(dvs)


def brute_force_attention(q, k, v):
    """Scalar pure-Python loops (tiny inputs only).  Returns nested lists (O, LSE).

    Independent restatement of s = q.k/sqrt(D), causal softmax, O = P v with
    query head h reading KV head h // G; used to cross-check ``attention_fwd``.
    """
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    q, k, v = q.tolist(), k.tolist(), v.tolist()
    scale = 1.0 / math.sqrt(D)
    out = [[[[0.0] * D for _ in range(T)] for _ in range(Hq)] for _ in range(B)]
    lse = [[[0.0] * T for _ in range(Hq)] for _ in range(B)]
    for b in range(B):
        for h in range(Hq):
            hk = h // G
            for i in range(T):
                s = []
                for j in range(i + 1):
                    acc = 0.0
                    for d in range(D):
                        acc += q[b][h][i][d] * k[b][hk][j][d]
                    s.append(acc * scale)
                m = max(s)
                e = [math.exp(x - m) for x in s]
                tot = sum(e)
                for d in range(D):
                    out[b][h][i][d] = sum(e[j] * v[b][hk][j][d] for j in range(i + 1)) / tot
                lse[b][h][i] = m + math.log(tot)
    return out, lse


def reference_outputs(q: Tensor, k: Tensor, v: Tensor, do: Tensor,
                      dtype: torch.dtype = torch.float32):
    """(O, LSE, dQ, dK, dV) from the explicit formulas, evaluated in ``dtype``.

    The forward output feeds the backward (as in the kernel, where dS uses the
    saved O through Delta).
    """
    o, lse = attention_fwd(q, k, v, dtype=dtype)
    dq, dk, dv = attention_bwd(q, k, v, o, do, lse, dtype=dtype)
    return o, lse, dq, dk, dv


def varlen_reference(q: Tensor, k: Tensor, v: Tensor, do: Tensor, cu_seqlens,
                     dtype: torch.dtype = torch.float32):
    """Packed variable-length attention: q/do [Hq, total, D], k/v [Hkv, total, D], every
    sequence s (rows cu[s]..cu[s+1]-1) attending causally within itself.  Returns
    (O, LSE [Hq, total], dQ, dK, dV) by running ``reference_outputs`` (the reference's
    causal attention, model.py:94-98 / kernels/flash_attn.py:12-217) on each sequence as
    a batch of one; rows of empty sequences do not exist.  Pinned in tests/test_oracle.py
    against dense attention over all rows with an explicit block-diagonal causal mask."""
    cu = [int(x) for x in cu_seqlens]
    outs = [torch.zeros_like(q, dtype=dtype), torch.zeros(q.shape[:2], dtype=dtype),
            torch.zeros_like(q, dtype=dtype), torch.zeros_like(k, dtype=dtype),
            torch.zeros_like(v, dtype=dtype)]
    for c0, c1 in zip(cu[:-1], cu[1:]):
        if c1 <= c0:
            continue
        o, lse, dq, dk, dv = reference_outputs(q[None, :, c0:c1], k[None, :, c0:c1],
                                               v[None, :, c0:c1], do[None, :, c0:c1], dtype=dtype)
        outs[0][:, c0:c1], outs[1][:, c0:c1] = o[0], lse[0]
        outs[2][:, c0:c1], outs[3][:, c0:c1], outs[4][:, c0:c1] = dq[0], dk[0], dv[0]
    return tuple(outs)


def decode_reference(q: Tensor, k_cache: Tensor, v_cache: Tensor, cache_seqlens,
                     dtype: torch.dtype = torch.float64):
    """KV-cache decode: q [B, Hq, Tq, D] are the newest Tq query rows of each sequence,
    row i at position L_b - Tq + i (L_b = cache_seqlens[b] clamped to the cache length)
    attending causally to cache keys 0 .. L_b - Tq + i -- the last Tq rows of the
    reference's causal attention (model.py:94-98).  Returns (O [B, Hq, Tq, D],
    LSE [B, Hq, Tq]); a row that sees no key gets O = 0, LSE = -inf.  Pinned in
    tests/test_oracle.py against the last rows of ``attention_fwd`` on full sequences."""
    B, Hq, Tq, D = q.shape
    Hkv, Lmax = k_cache.shape[1], k_cache.shape[2]
    G = Hq // Hkv
    o = torch.zeros((B, Hq, Tq, D), dtype=dtype)
    lse = torch.full((B, Hq, Tq), float("-inf"), dtype=dtype)
    for b in range(B):
        L = min(max(int(cache_seqlens[b]), 0), Lmax)
        if L == 0:
            continue
        k = k_cache[b, :, :L].to(dtype).repeat_interleave(G, 0)
        v = v_cache[b, :, :L].to(dtype).repeat_interleave(G, 0)
        s = q[b].to(dtype) @ k.transpose(-1, -2) / math.sqrt(D)
        pos = torch.arange(Tq)[:, None] + (L - Tq)
        s = s.masked_fill(torch.arange(L)[None, :] > pos, float("-inf"))
        seen = pos[:, 0] >= 0
        if not bool(seen.any()):
            continue
        lse_b = torch.logsumexp(s, -1)
        p = torch.exp(s - lse_b[..., None])
        o[b][:, seen] = (p @ v)[:, seen]
        lse[b][:, seen] = lse_b[:, seen]
    return o, lse


def max_abs(a: Tensor, b: Tensor) -> float:
    """max |a - b| in fp64 (NaN anywhere counts as infinite error)."""
    d = (a.detach().double().cpu() - b.detach().double().cpu()).abs()
    if torch.isnan(d).any():
        return float("inf")
    return float(d.max()) if d.numel() else 0.0


# Parity tolerances (max-abs against this oracle) from the workload specification:
# O, dQ, dK, dV within 2e-2 for bf16 inputs and 1e-5 for fp32; LSE within 1e-3.
TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-5}
TOL_LSE = 1e-3
