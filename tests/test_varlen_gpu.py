"""GPU tests of packed variable-length attention (cu_seqlens) against the batched kernels
and the CPU oracle.

* each sequence's O / LSE / dQ / dK / dV from the varlen launch are bitwise those of the
  batched launch on that sequence alone (B = 1, T = its length): the same tiles run the
  same arithmetic, only the work-item mapping differs;
* the packed result matches oracle.eager_attention.varlen_reference (block-diagonal
  causal attention, fp32) within the attention tolerances;
* empty sequences, length-1 sequences, tile-boundary lengths, a 4500-token sequence, GQA,
  both head dims;
  rows of sequences with invalid bounds are left unwritten; opcheck and autograd.
"""


import pytest
import torch

from helpers import announce, assert_close_abs
from oracle.eager_attention import TOL, TOL_LSE, varlen_reference
from tinytrain_amd.kernels.flash_attn import (_backward, _forward, flash_attn_varlen,
                                              flash_attn_varlen_bwd, flash_attn_varlen_fwd)

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    ([1, 127, 128, 129, 300, 64], 8, 2, 64),
    ([5, 0, 256, 1000, 3], 4, 4, 128),
    ([513, 77], 16, 8, 128),
    # long rows at D = 64 (the batched kernels there have no 256-row form, so bitwise
    # equality to the per-sequence launch holds at any length)
    ([4500, 1, 2047, 129], 4, 2, 64),
]


def _inputs(lens, Hq, Hkv, D, seed=0):
    total = sum(lens)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Hq, total, D, generator=g)
    k = torch.randn(Hkv, total, D, generator=g)
    q = q / q.pow(2).mean(-1, keepdim=True).sqrt()
    k = k / k.pow(2).mean(-1, keepdim=True).sqrt()
    v = torch.randn(Hkv, total, D, generator=g)
    do = torch.randn(Hq, total, D, generator=g) * 1e-2
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    return [t.to(torch.bfloat16) for t in (q, k, v, do)] + [cu]


@pytest.mark.parametrize("lens,Hq,Hkv,D", CASES)
def test_varlen_bitwise_equals_per_sequence(lens, Hq, Hkv, D):
    announce(f"varlen vs per-sequence lens={lens} Hq={Hq} Hkv={Hkv} D={D}")
    q, k, v, do, cu = _inputs(lens, Hq, Hkv, D)
    qd, kd, vd, dod, cud = (t.to(DEV) for t in (q, k, v, do, cu))
    o, M = flash_attn_varlen_fwd(qd, kd, vd, cud, max(lens))
    dq, dk, dv = flash_attn_varlen_bwd(qd, kd, vd, o, dod, M, cud, max(lens))
    torch.cuda.synchronize()
    for c0, c1 in zip(cu[:-1].tolist(), cu[1:].tolist()):
        if c1 == c0:
            continue
        sl = lambda t: t[:, c0:c1].unsqueeze(0).contiguous()
        o1, M1 = _forward(sl(qd), sl(kd), sl(vd))
        dq1, dk1, dv1 = _backward(sl(qd), sl(kd), sl(vd), o1, sl(dod), M1)
        torch.cuda.synchronize()
        for name, a, b in (("o", o, o1), ("lse", M, M1), ("dq", dq, dq1), ("dk", dk, dk1),
                           ("dv", dv, dv1)):
            assert torch.equal(a[:, c0:c1], b[0]), f"{name} differs for sequence [{c0}, {c1})"


@pytest.mark.parametrize("lens,Hq,Hkv,D", CASES)
def test_varlen_matches_oracle(lens, Hq, Hkv, D):
    announce(f"varlen vs oracle lens={lens} Hq={Hq} Hkv={Hkv} D={D}")
    q, k, v, do, cu = _inputs(lens, Hq, Hkv, D, seed=1)
    want = varlen_reference(q.float(), k.float(), v.float(), do.float(), cu.tolist())
    qd, kd, vd, dod, cud = (t.to(DEV) for t in (q, k, v, do, cu))
    o, M = flash_attn_varlen_fwd(qd, kd, vd, cud, max(lens))
    dq, dk, dv = flash_attn_varlen_bwd(qd, kd, vd, o, dod, M, cud, max(lens))
    torch.cuda.synchronize()
    tol = TOL[torch.bfloat16]
    assert_close_abs("O", o.cpu(), want[0], tol)
    assert_close_abs("LSE", M.cpu(), want[1], TOL_LSE)
    for name, a, b in (("dQ", dq, want[2]), ("dK", dk, want[3]), ("dV", dv, want[4])):
        assert_close_abs(name, a.cpu(), b, tol)


def test_invalid_sequence_bounds_are_skipped():
    """Sequences whose bounds leave 0..total or decrease are skipped: the launch completes,
    reads nothing outside the tensors, and the valid sequence's rows are exact."""
    announce("varlen invalid bounds skipped")
    q, k, v, do, cu = _inputs([64, 64, 64], 4, 2, 64)
    bad = torch.tensor([0, 64, 300, 192], dtype=torch.int32)  # [64, 300) and [300, 192) invalid
    qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
    o, M = flash_attn_varlen_fwd(qd, kd, vd, bad.to(DEV), 64)
    dq, dk, dv = flash_attn_varlen_bwd(qd, kd, vd, o, dod, M, bad.to(DEV), 64)
    ref_o, ref_M = flash_attn_varlen_fwd(qd, kd, vd, cu.to(DEV), 64)
    ref = flash_attn_varlen_bwd(qd, kd, vd, ref_o, dod, ref_M, cu.to(DEV), 64)
    torch.cuda.synchronize()
    assert torch.equal(o[:, :64], ref_o[:, :64]) and torch.equal(M[:, :64], ref_M[:, :64])
    for a, b in zip((dq, dk, dv), ref):
        assert torch.equal(a[:, :64], b[:, :64])


def test_varlen_autograd_and_opcheck():
    announce("varlen autograd + opcheck")
    q, k, v, do, cu = (t.to(DEV) for t in _inputs([100, 28, 200], 4, 2, 64))
    qr, kr, vr = (t.clone().requires_grad_() for t in (q, k, v))
    o = flash_attn_varlen(qr, kr, vr, cu, 200)
    o.backward(do)
    o2, M = flash_attn_varlen_fwd(q, k, v, cu, 200)
    dq, dk, dv = flash_attn_varlen_bwd(q, k, v, o2, do, M, cu, 200)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(qr.grad, dq) and torch.equal(kr.grad, dk)
    assert torch.equal(vr.grad, dv)
    torch.library.opcheck(flash_attn_varlen_fwd, (q, k, v, cu, 200),
                          test_utils=("test_schema", "test_faketensor"))
    torch.library.opcheck(flash_attn_varlen_bwd, (q, k, v, o2, do, M, cu, 200),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.parametrize("D", [64, 128])
def test_sequence_longer_than_max_seqlen(D):
    """A sequence longer than max_seqlen is processed as its first max_seqlen tokens by
    all three kernels: those rows of o, lse, dq, dk, dv are bitwise the batched result on
    the truncated sequence, and its later rows stay unwritten (NaN poison survives)."""
    import math

    from tinytrain_amd import _lib

    lens, max_seqlen, Hq, Hkv = [300, 100], 200, 4, 2
    announce(f"varlen understated max_seqlen lens={lens} max_seqlen={max_seqlen} D={D}")
    q, k, v, do, cu = (t.to(DEV) for t in _inputs(lens, Hq, Hkv, D, seed=4))
    total = sum(lens)
    nan = float("nan")
    o, dq = torch.full_like(q, nan), torch.full_like(q, nan)
    dk, dv = torch.full_like(k, nan), torch.full_like(v, nan)
    M = torch.full((Hq, total), nan, device=DEV)
    delta = torch.full((Hq, total), nan, device=DEV)
    lib, s, sc = _lib.load(), torch.cuda.current_stream().cuda_stream, 1.0 / math.sqrt(D)
    _lib.check(lib.ttfa_varlen_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                   M.data_ptr(), cu.data_ptr(), len(lens), total, max_seqlen,
                                   Hq, Hkv, D, _lib.TTFA_BF16, sc, s))
    _lib.check(lib.ttfa_varlen_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                   do.data_ptr(), M.data_ptr(), delta.data_ptr(), dq.data_ptr(),
                                   dk.data_ptr(), dv.data_ptr(), cu.data_ptr(), len(lens), total,
                                   max_seqlen, Hq, Hkv, D, _lib.TTFA_BF16, sc, s))
    torch.cuda.synchronize()
    for c0, n in ((0, max_seqlen), (lens[0], lens[1])):  # written rows of each sequence
        sl = lambda t: t[:, c0:c0 + n].unsqueeze(0).contiguous()
        o1, M1 = _forward(sl(q), sl(k), sl(v))
        dq1, dk1, dv1 = _backward(sl(q), sl(k), sl(v), o1, sl(do), M1)
        torch.cuda.synchronize()
        for name, a, b in (("o", o, o1), ("lse", M, M1), ("dq", dq, dq1), ("dk", dk, dk1),
                           ("dv", dv, dv1)):
            assert torch.equal(a[:, c0:c0 + n], b[0]), f"{name} rows [{c0}, {c0 + n}) differ"
    for name, t in (("o", o), ("lse", M), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.isnan(t[:, max_seqlen:lens[0]].float()).all(), \
            f"{name}: rows past max_seqlen of the long sequence were written"
