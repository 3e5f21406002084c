"""GPU parity at the longest rows: T = 65536 at D = 64 (512 row tiles of 128) and a ragged
T = 40001 at D = 128 (the 256-row forward and dQ kernels), one sequence with two query heads
on one KV head.

A full fp64 oracle at these lengths is out of reach on the CPU in a test, so each output is
checked against what defines it:

* O and LSE of every row: the oracle's chunked forward (attention_fwd) in fp32;
* dQ of sampled rows and dK / dV of sampled keys, in fp64 from their definitions
  (attention_bwd_rows / attention_bwd_keys, pinned against the full backward in
  tests/test_oracle.py), with the oracle's O and LSE for every row.

Inputs follow the configurations' distribution (unit-RMS q and k, v ~ N(0, 1),
dO ~ N(0, 1) * 1e-2), drawn on the CPU.  Besides the max-abs bound of every other parity test,
each gradient is held to 2% of its own largest magnitude, since at this dO scale the
gradients sit far below the absolute bound.
"""

import pytest
import torch

from helpers import announce, assert_close_abs
from oracle.eager_attention import (TOL, TOL_LSE, attention_bwd_keys, attention_bwd_rows,
                                    attention_fwd)
from tinytrain_amd.workloads import unit_rms
from tinytrain_amd.kernels.flash_attn import _backward, _forward

pytestmark = pytest.mark.gpu

REL = 2e-2


def _inputs(Hq, Hkv, T, D, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    q = unit_rms(torch.randn(1, Hq, T, D, generator=g))
    k = unit_rms(torch.randn(1, Hkv, T, D, generator=g))
    v = torch.randn(1, Hkv, T, D, generator=g)
    do = torch.randn(1, Hq, T, D, generator=g) * 1e-2
    return tuple(t.to(torch.bfloat16).contiguous() for t in (q, k, v, do))


def _sample(T, fixed, n, seed):
    g = torch.Generator().manual_seed(seed)
    idx = {t for t in fixed if 0 <= t < T}
    idx.update(torch.randint(0, T, (n,), generator=g).tolist())
    return sorted(idx)


def _check(name, got, want, ctx):
    assert_close_abs(name, got, want, TOL[torch.bfloat16], ctx)
    scale = want.abs().max().item()
    err = (got.double() - want).abs().max().item()
    assert err <= REL * scale, f"{name}: max|err| = {err:.3e} > {REL} * {scale:.3e} {ctx}"


@pytest.mark.parametrize("Hq, Hkv, T, D", [
    (2, 1, 65536, 64),    # 512 row tiles; every pass's longest items
    (2, 1, 40001, 128),   # T > 3840 and ragged: the 256-row forward and dQ kernels
])
def test_long_rows(Hq, Hkv, T, D):
    announce(f"long rows Hq={Hq} Hkv={Hkv} T={T} D={D}")
    q, k, v, do = _inputs(Hq, Hkv, T, D, seed=T + D)
    qd, kd, vd, dod = (t.to("cuda") for t in (q, k, v, do))
    o, lse = _forward(qd, kd, vd)
    dq, dk, dv = _backward(qd, kd, vd, o, dod, lse)
    torch.cuda.synchronize()
    o, lse, dq, dk, dv = (t.cpu() for t in (o, lse, dq, dk, dv))
    for t in (o, lse, dq, dk, dv):
        assert torch.isfinite(t.float()).all()

    o_ref, lse_ref = attention_fwd(q, k, v, dtype=torch.float32)
    assert_close_abs("o", o, o_ref, TOL[torch.bfloat16], f"[T={T} D={D} every row]")
    assert_close_abs("lse", lse, lse_ref, TOL_LSE, f"[T={T} D={D} every row]")

    edges = (0, 1, 31, 32, 127, 128, 255, 256, 4095, 4096, T // 2, T - 257, T - 129, T - 128,
             T - 2, T - 1)
    rows = _sample(T, edges, 8, seed=T)
    for h in range(Hq):
        want = attention_bwd_rows(q, k, v, do, o_ref, lse_ref, 0, h, rows)
        _check("dq", dq[0, h, rows], want, f"[T={T} D={D} head {h} rows {rows}]")
    keys = _sample(T, edges, 8, seed=T + 1)
    for hk in range(Hkv):
        want_k, want_v = attention_bwd_keys(q, k, v, do, o_ref, lse_ref, 0, hk, keys)
        _check("dk", dk[0, hk, keys], want_k, f"[T={T} D={D} kv head {hk} keys {keys}]")
        _check("dv", dv[0, hk, keys], want_v, f"[T={T} D={D} kv head {hk} keys {keys}]")
