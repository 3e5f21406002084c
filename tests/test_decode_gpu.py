"""GPU tests of KV-cache decode attention against the CPU oracle and the forward kernel.

* outputs match oracle.eager_attention.decode_reference (the last Tq rows of causal
  attention, fp64) within the attention tolerances, for MHA / GQA, both head dims,
  Tq = 1 and Tq > 1, per-batch cache lengths including lengths shorter than Tq (rows
  that see no key: O = 0, LSE = -inf), 1, and the full cache;
* decoding the last rows of a sequence agrees with the batched forward kernel on the
  whole sequence;
* run-to-run bitwise determinism and the torch.library op checks;
* a workspace reused across shapes with leftovers in it, and HIP-graph replays with new
  inputs, both bitwise equal to fresh eager calls.
"""

import pytest
import torch

from helpers import announce, assert_close_abs
from oracle.eager_attention import TOL, TOL_LSE, decode_reference
from tinytrain_amd.kernels.decode import flash_attn_decode
from tinytrain_amd.kernels.flash_attn import _forward

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # B, Hq, Hkv, Tq, Lmax, D, lens
    (4, 16, 8, 1, 4096, 128, [4096, 1, 33, 2500]),
    (2, 8, 2, 4, 300, 64, [300, 5]),
    (3, 4, 4, 3, 1000, 128, [2, 999, 64]),
    (1, 32, 4, 4, 128, 64, [128]),          # 8 * 4 = 32 query rows per KV head
    (8, 12, 12, 1, 2048, 64, [2048, 1500, 1024, 511, 64, 33, 32, 31]),
]


def _inputs(B, Hq, Hkv, Tq, Lmax, D, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Tq, D, generator=g)
    q = q / q.pow(2).mean(-1, keepdim=True).sqrt()
    k = torch.randn(B, Hkv, Lmax, D, generator=g)
    k = k / k.pow(2).mean(-1, keepdim=True).sqrt()
    v = torch.randn(B, Hkv, Lmax, D, generator=g)
    return [t.to(torch.bfloat16) for t in (q, k, v)]


@pytest.mark.parametrize("B,Hq,Hkv,Tq,Lmax,D,lens", CASES)
def test_decode_matches_oracle(B, Hq, Hkv, Tq, Lmax, D, lens):
    announce(f"decode B={B} Hq={Hq} Hkv={Hkv} Tq={Tq} Lmax={Lmax} D={D} lens={lens}")
    q, k, v = _inputs(B, Hq, Hkv, Tq, Lmax, D)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    want_o, want_lse = decode_reference(q, k, v, lens)
    o, lse = flash_attn_decode(q.to(DEV), k.to(DEV), v.to(DEV), lens_t.to(DEV))
    torch.cuda.synchronize()
    assert_close_abs("O", o.cpu(), want_o, TOL[torch.bfloat16])
    fin = torch.isfinite(want_lse)
    assert torch.equal(torch.isfinite(lse.cpu()), fin)
    assert_close_abs("LSE", lse.cpu()[fin], want_lse[fin], TOL_LSE)


def test_decode_agrees_with_forward_kernel():
    announce("decode vs batched forward last rows")
    B, Hq, Hkv, T, D, Tq = 2, 8, 2, 700, 128, 2
    g = torch.Generator().manual_seed(1)
    q = torch.randn(B, Hq, T, D, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).to(DEV)
    o_full, lse_full = _forward(q, k, v)
    lens = torch.full((B,), T, dtype=torch.int32, device=DEV)
    o, lse = flash_attn_decode(q[:, :, T - Tq:].contiguous(), k, v, lens)
    torch.cuda.synchronize()
    assert_close_abs("O", o, o_full[:, :, T - Tq:], TOL[torch.bfloat16])
    assert_close_abs("LSE", lse, lse_full[:, :, T - Tq:], TOL_LSE)


@pytest.mark.parametrize("B, L", [(32, 4096), (1, 16384), (128, 1024)])
def test_decode_bench_shapes_match_forward(B, L):
    """At the decode bench's shapes (Hq 16, Hkv 8, D 128; hundreds of key splits per row
    at B=1), the decoded row of every batch equals row cache_len-1 of the batched forward
    kernel over the whole cache, for per-batch cache lengths."""
    announce(f"decode bench shape B={B} L={L}")
    Hq, Hkv, D = 16, 8, 128
    g = torch.Generator(device=DEV).manual_seed(3)

    def unit_rms(t):
        return (t / t.pow(2).mean(-1, keepdim=True).sqrt()).to(torch.bfloat16)

    q = unit_rms(torch.randn(B, Hq, L, D, device=DEV, generator=g))
    k = unit_rms(torch.randn(B, Hkv, L, D, device=DEV, generator=g))
    v = torch.randn(B, Hkv, L, D, device=DEV, generator=g).to(torch.bfloat16)
    lens = torch.randint(1, L + 1, (B,), device=DEV, generator=g, dtype=torch.int32)
    lens[0] = L
    o_full, lse_full = _forward(q, k, v)
    rows = (lens.long() - 1).view(B, 1, 1, 1).expand(B, Hq, 1, D)
    qd = torch.gather(q, 2, rows).contiguous()
    o, lse = flash_attn_decode(qd, k, v, lens)
    want_o = torch.gather(o_full, 2, rows)
    want_lse = torch.gather(lse_full, 2, (lens.long() - 1).view(B, 1, 1).expand(B, Hq, 1))
    torch.cuda.synchronize()
    assert_close_abs("O", o, want_o, TOL[torch.bfloat16])
    assert_close_abs("LSE", lse, want_lse, TOL_LSE)


def test_decode_deterministic_and_opcheck():
    announce("decode determinism + opcheck")
    q, k, v = (t.to(DEV) for t in _inputs(4, 8, 2, 2, 1024, 64, seed=2))
    lens = torch.tensor([1024, 700, 3, 1], dtype=torch.int32, device=DEV)
    a = flash_attn_decode(q, k, v, lens)
    b = flash_attn_decode(q, k, v, lens)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    torch.library.opcheck(flash_attn_decode, (q, k, v, lens),
                          test_utils=("test_schema", "test_faketensor"))


def test_decode_shared_workspace_with_leftovers():
    """One workspace reused by calls of different shapes through the C ABI, first filled
    with random bits: every call equals a call of the op on a fresh workspace, bitwise
    (nothing a call reads from the workspace was left there by another)."""
    import math

    from tinytrain_amd import _lib

    announce("decode shared workspace with leftovers")
    lib = _lib.load()
    shapes = [(1, 16, 8, 1, 16384, 128, [16384]), (4, 8, 2, 2, 1024, 64, [1024, 700, 3, 1]),
              (128, 16, 8, 1, 1024, 128, None), (2, 12, 12, 1, 5000, 64, [4999, 2048])]
    need = max(lib.ttfa_decode_workspace_bytes(B, Hq, Hkv, Tq, L, D)
               for B, Hq, Hkv, Tq, L, D, _ in shapes)
    ws = torch.randint(-2**62, 2**62, (need // 8 + 2,), dtype=torch.int64, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    for rep in range(2):
        for i, (B, Hq, Hkv, Tq, L, D, lens) in enumerate(shapes):
            q, k, v = (t.to(DEV) for t in _inputs(B, Hq, Hkv, Tq, L, D, seed=10 * i + rep))
            if lens is None:
                lens = [L - 7 * j for j in range(B)]
            lens_t = torch.tensor(lens, dtype=torch.int32, device=DEV)
            want_o, want_lse = flash_attn_decode(q, k, v, lens_t)
            o, lse = torch.empty_like(q), torch.empty(B, Hq, Tq, device=DEV)
            _lib.check(lib.ttfa_decode_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                           lens_t.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                           ws.data_ptr(), B, Hq, Hkv, Tq, L, D, _lib.TTFA_BF16,
                                           1.0 / math.sqrt(D), stream))
            torch.cuda.synchronize()
            assert torch.equal(o, want_o), (rep, i)
            assert torch.equal(lse, want_lse), (rep, i)


def test_decode_graph_replays():
    """flash_attn_decode captured in a HIP graph (16 key splits per row) and replayed with
    new cache contents and lengths between the replays (eager work and synchronisations in
    between): each replay equals the eager op on the same inputs, bitwise."""
    announce("decode graph replays")
    B, Hq, Hkv, Tq, L, D = 2, 16, 8, 1, 8192, 128
    q_s, k_s, v_s = (t.to(DEV) for t in _inputs(B, Hq, Hkv, Tq, L, D, seed=20))
    lens_s = torch.tensor([L, 5000], dtype=torch.int32, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        flash_attn_decode(q_s, k_s, v_s, lens_s)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_s, lse_s = flash_attn_decode(q_s, k_s, v_s, lens_s)
    for r in range(4):
        q, k, v = (t.to(DEV) for t in _inputs(B, Hq, Hkv, Tq, L, D, seed=21 + r))
        q_s.copy_(q)
        k_s.copy_(k)
        v_s.copy_(v)
        lens_s.copy_(torch.tensor([L - 100 * r, 3000 + 7 * r], dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        want_o, want_lse = flash_attn_decode(q_s, k_s, v_s, lens_s)
        torch.cuda.synchronize()
        assert torch.equal(o_s, want_o), r
        assert torch.equal(lse_s, want_lse), r
