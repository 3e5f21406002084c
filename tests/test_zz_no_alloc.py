"""ttfa_bwd_static: the backward without a delta_ws argument (Delta in a library-owned
static device array), for callers that cannot allocate.  It has no reference counterpart.

* CPU: argument validation, including the size limit, returns before any HIP call;
* GPU: two calls in a row, the second with a smaller input, each bitwise equal to ttfa_bwd
  on the same input (same kernels; only where Delta lives differs).
"""

import math

import pytest
import torch

from helpers import announce
from tinytrain_amd import _lib
from tinytrain_amd.workloads import make_custom

needs_lib = pytest.mark.skipif(not _lib.LIB_PATH.exists(),
                               reason="libttfa.so not built (python -m tinytrain_amd.build)")


def _call_static(lib, ptrs, B, Hq, Hkv, T, D, dt=_lib.TTFA_BF16, scale=0.125, stream=None):
    return lib.ttfa_bwd_static(*ptrs, B, Hq, Hkv, T, D, dt, scale, stream)


@needs_lib
def test_static_size_limit_and_pointer_checks():
    lib = _lib.load()
    p = [16] * 9  # aligned non-null stand-ins: validation returns before they are touched
    rows = _lib.BWD_STATIC_MAX_ROWS
    assert _call_static(lib, p, 1, 16, 8, rows // 16 + 1, 64) == _lib.E_SCRATCH
    assert _call_static(lib, p, 4, 16, 8, 16384 + 1, 128) == _lib.E_SCRATCH
    assert _call_static(lib, p, 1, 16, 8, 65537, 64) == _lib.E_SCRATCH
    assert _call_static(lib, p, 1, 12, 5, 64, 64) == _lib.E_GROUP
    for i in range(9):
        bad = list(p)
        bad[i] = None
        assert _call_static(lib, bad, 1, 4, 2, 64, 64) == _lib.E_NULL
        bad[i] = 24
        assert _call_static(lib, bad, 1, 4, 2, 64, 64) == _lib.E_ALIGN
    assert "TTFA_BWD_STATIC_MAX_ROWS" in _lib.strerror(_lib.E_SCRATCH)


def _bwd_both(B, Hq, Hkv, T, D, dtype, seed):
    """(ttfa_bwd outputs, ttfa_bwd_static outputs) on one seeded input."""
    from tinytrain_amd.kernels.flash_attn import _forward

    q, k, v, do = (t.to("cuda") for t in make_custom(B, Hq, Hkv, T, D, dtype, seed=seed,
                                                     do_scale=1e-2))
    o, M = _forward(q, k, v)
    lib, s = _lib.load(), torch.cuda.current_stream().cuda_stream
    dt = _lib.TTFA_BF16 if dtype == torch.bfloat16 else _lib.TTFA_F32
    sc = 1.0 / math.sqrt(D)
    nan = float("nan")
    outs = []
    for static in (False, True):
        dq, dk, dv = torch.full_like(q, nan), torch.full_like(k, nan), torch.full_like(v, nan)
        common = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
                  M.data_ptr())
        if static:
            rc = lib.ttfa_bwd_static(*common, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, Hq,
                                     Hkv, T, D, dt, sc, s)
        else:
            delta = torch.empty((B, Hq, T), device="cuda", dtype=torch.float32)
            rc = lib.ttfa_bwd(*common, delta.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                              dv.data_ptr(), B, Hq, Hkv, T, D, dt, sc, s)
        _lib.check(rc)
        outs.append((dq, dk, dv))
    torch.cuda.synchronize()
    return outs


@pytest.mark.gpu
def test_static_matches_workspace_entry_point_twice():
    """Two calls in a row on one GPU, the second smaller: each equals ttfa_bwd bitwise."""
    cases = [(2, 6, 2, 700, 64, torch.bfloat16, 1), (1, 4, 4, 77, 128, torch.bfloat16, 2),
             (1, 2, 1, 45, 64, torch.float32, 3)]
    for B, Hq, Hkv, T, D, dtype, seed in cases:
        announce(f"ttfa_bwd_static B={B} Hq={Hq} Hkv={Hkv} T={T} D={D} {dtype}")
        ref, got = _bwd_both(B, Hq, Hkv, T, D, dtype, seed)
        for name, a, b in zip(("dq", "dk", "dv"), got, ref):
            assert torch.isfinite(a.float()).all(), f"{name}: unwritten elements"
            assert torch.equal(a, b), f"{name} differs from ttfa_bwd (B={B} T={T} D={D})"
