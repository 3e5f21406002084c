"""CPU checks that pin the attention oracle (oracle/eager_attention.py).

The reference publishes no frozen attention vectors, so the oracle is pinned by
(1) agreement of independent implementations: torch's SDPA library routine
(the reference's eager path, model.py:94-98), explicit fp64 matmuls, and scalar
Python loops; (2) closed forms and invariants the mathematics fixes; (3) autograd
and finite differences for every backward formula; (4) planted mistakes (a wrong GQA
head map, a dropped Delta term, a transposed operand) that these checks must catch.
"""

import math

import pytest
import torch

from oracle.eager_attention import (attention_bwd, attention_bwd_keys, attention_bwd_rows,
                                    attention_delta, attention_fwd,
                                    brute_force_attention, eager_attention,
                                    eager_attention_grads, max_abs, reference_outputs,
                                    varlen_reference)
from tinytrain_amd.workloads import CONFIGS, make_custom, make_inputs


def _rand(B, Hq, Hkv, T, D, seed=0, dtype=torch.float64):
    g = torch.Generator("cpu").manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g, dtype=dtype)
    return mk(B, Hq, T, D), mk(B, Hkv, T, D), mk(B, Hkv, T, D), mk(B, Hq, T, D)


@pytest.mark.parametrize("B, Hq, Hkv, T, D", [(2, 4, 2, 37, 64), (1, 6, 2, 70, 128),
                                              (1, 2, 2, 1, 64)])
def test_explicit_fwd_matches_sdpa(B, Hq, Hkv, T, D):
    q, k, v, _ = _rand(B, Hq, Hkv, T, D)
    o_sdpa = eager_attention(q, k, v)            # fp32 library routine
    o, _ = attention_fwd(q, k, v)                # fp64 explicit
    assert max_abs(o_sdpa, o) < 1e-5


def test_brute_force_loops_match():
    q, k, v, _ = _rand(1, 4, 2, 6, 8, seed=3)
    o_bf, lse_bf = brute_force_attention(q, k, v)
    o, lse = attention_fwd(q, k, v)
    assert max_abs(torch.tensor(o_bf, dtype=torch.float64), o) < 1e-12
    assert max_abs(torch.tensor(lse_bf, dtype=torch.float64), lse) < 1e-12


def test_single_row_closed_form():
    # T=1: softmax over one key gives O = v, LSE = q.k * scale.
    q, k, v, _ = _rand(2, 4, 2, 1, 64, seed=4)
    o, lse = attention_fwd(q, k, v)
    ke, ve = k.repeat_interleave(2, 1), v.repeat_interleave(2, 1)
    assert max_abs(o, ve) < 1e-14
    assert max_abs(lse, (q * ke).sum(-1) / 8.0) < 1e-12


def test_zero_query_is_running_mean():
    # q = 0: every visible score is 0, so O_i = mean_{j<=i} v_j and LSE_i = ln(i+1).
    _, k, v, _ = _rand(1, 2, 1, 40, 64, seed=5)
    q = torch.zeros(1, 2, 40, 64, dtype=torch.float64)
    o, lse = attention_fwd(q, k, v)
    csum = v.cumsum(dim=2) / torch.arange(1, 41, dtype=torch.float64)[:, None]
    assert max_abs(o, csum.expand(1, 2, 40, 64)) < 1e-12
    assert max_abs(lse, torch.log(torch.arange(1, 41, dtype=torch.float64)).expand(1, 2, 40)) < 1e-12


def test_lse_normalises_probabilities():
    q, k, v, _ = _rand(1, 2, 2, 50, 64, seed=6)
    _, lse = attention_fwd(q, k, v)
    s = q @ k.transpose(-1, -2) / 8.0
    s = s.masked_fill(torch.ones(50, 50).triu(1).bool(), float("-inf"))
    tot = torch.exp(s - lse[..., None]).sum(-1)
    assert max_abs(tot, torch.ones_like(tot)) < 1e-12


def test_causality():
    # Changing the last key/value row changes only the last output row
    # (the reference's tests/test_model.py:49-63 checks this on the module).
    q, k, v, _ = _rand(1, 4, 2, 30, 64, seed=7)
    o1, _ = attention_fwd(q, k, v)
    k2, v2 = k.clone(), v.clone()
    k2[:, :, -1] += 1.0
    v2[:, :, -1] -= 2.0
    o2, _ = attention_fwd(q, k2, v2)
    assert max_abs(o1[:, :, :-1], o2[:, :, :-1]) == 0.0
    assert max_abs(o1[:, :, -1], o2[:, :, -1]) > 1e-3


def test_gqa_equals_expanded_heads():
    # model.py:96-97 (repeat_interleave) and tests/test_model.py:174-200: grouped heads
    # equal explicit expansion; dK/dV equal the sum over the group.
    q, k, v, do = _rand(2, 6, 2, 25, 64, seed=8)
    o, lse = attention_fwd(q, k, v)
    ke, ve = k.repeat_interleave(3, 1), v.repeat_interleave(3, 1)
    o_e, lse_e = attention_fwd(q, ke, ve)
    assert max_abs(o, o_e) == 0.0 and max_abs(lse, lse_e) == 0.0
    dq, dk, dv = attention_bwd(q, k, v, o, do, lse)
    dq_e, dk_e, dv_e = attention_bwd(q, ke, ve, o_e, do, lse_e)
    assert max_abs(dq, dq_e) < 1e-12
    assert max_abs(dk, dk_e.view(2, 2, 3, 25, 64).sum(2)) < 1e-12
    assert max_abs(dv, dv_e.view(2, 2, 3, 25, 64).sum(2)) < 1e-12


def test_bwd_formulas_match_autograd_fp64():
    # attention_bwd's hand-written formulas vs autograd through the explicit forward.
    q, k, v, do = _rand(2, 4, 2, 33, 64, seed=9)
    qr, kr, vr = (t.clone().requires_grad_() for t in (q, k, v))
    o_ad, _ = attention_fwd(qr, kr, vr)
    o_ad.backward(do)
    o, lse = attention_fwd(q, k, v)
    dq, dk, dv = attention_bwd(q, k, v, o, do, lse)
    assert max_abs(dq, qr.grad) < 1e-12
    assert max_abs(dk, kr.grad) < 1e-12
    assert max_abs(dv, vr.grad) < 1e-12


def test_bwd_matches_sdpa_autograd():
    # The contract: gradients of the eager path (repeat_interleave + SDPA, fp32).
    q, k, v, do = _rand(1, 4, 2, 45, 128, seed=10)
    o_e, dq_e, dk_e, dv_e = eager_attention_grads(q, k, v, do)
    o, lse = attention_fwd(q, k, v)
    dq, dk, dv = attention_bwd(q, k, v, o, do, lse)
    for a, b in ((o, o_e), (dq, dq_e), (dk, dk_e), (dv, dv_e)):
        assert max_abs(a, b) < 2e-5


def test_forward_gradcheck_finite_differences():
    # Finite differences fix the derivative independently of how either side is written.
    q, k, v, _ = _rand(1, 2, 1, 5, 4, seed=11)
    q, k, v = (t.requires_grad_() for t in (q, k, v))
    assert torch.autograd.gradcheck(lambda a, b, c: attention_fwd(a, b, c)[0], (q, k, v))
    assert torch.autograd.gradcheck(lambda a, b, c: attention_fwd(a, b, c)[1], (q, k, v))


def test_delta_is_rowsum():
    o = torch.arange(12, dtype=torch.float64).view(1, 1, 3, 4)
    do = torch.ones_like(o) * 2
    assert attention_delta(o, do).tolist() == [[[12.0, 44.0, 76.0]]]


def test_chunked_rows_match_unchunked(monkeypatch):
    # The oracle evaluates long rows in chunks of query rows; the chunking is exact.
    import oracle.eager_attention as ea
    q, k, v, do = _rand(1, 2, 1, 70, 64, seed=12)
    full = reference_outputs(q, k, v, do, dtype=torch.float64)
    monkeypatch.setattr(ea, "_CHUNK", 16)
    chunked = reference_outputs(q, k, v, do, dtype=torch.float64)
    for a, b in zip(full, chunked):
        assert max_abs(a, b) < 1e-12


# ------------------------------------------------------- planted mistakes are caught
def _fwd_wrong_head_map(q, k, v):
    """attention_fwd with query head h reading KV head h % Hkv (instead of h // G)."""
    g = q.shape[1] // k.shape[1]
    return attention_fwd(q, k.repeat(1, g, 1, 1), v.repeat(1, g, 1, 1))


def test_planted_wrong_head_map_is_caught():
    q, k, v, _ = _rand(1, 4, 2, 20, 64, seed=13)
    o_bad, _ = _fwd_wrong_head_map(q, k, v)
    assert max_abs(o_bad, eager_attention(q, k, v)) > 1e-2


def test_planted_dropped_delta_is_caught():
    q, k, v, do = _rand(1, 2, 2, 20, 64, seed=14)
    o, lse = attention_fwd(q, k, v)
    dq_bad, _, _ = attention_bwd(q, k, v, torch.zeros_like(o), do, lse)  # Delta = 0
    _, dq_e, _, _ = eager_attention_grads(q, k, v, do)
    assert max_abs(dq_bad, dq_e) > 1e-3


def test_planted_swapped_kv_is_caught():
    # The reference's mutation list: swapping k and v must fail the output check.
    q, k, v, _ = _rand(1, 2, 2, 20, 64, seed=15)
    o_bad, _ = attention_fwd(q, v, k)
    assert max_abs(o_bad, eager_attention(q, k, v)) > 1e-2


@pytest.mark.parametrize("Hq, Hkv, T, D", [(4, 2, 45, 64), (3, 1, 33, 128)])
def test_sampled_rows_and_keys_match_full_backward(Hq, Hkv, T, D):
    """The per-row dQ and per-key dK / dV forms (used where the full backward is too
    slow) equal the full backward on every row and key, GQA included."""
    q, k, v, do = _rand(2, Hq, Hkv, T, D, seed=21)
    o, lse = attention_fwd(q, k, v)
    dq, dk, dv = attention_bwd(q, k, v, o, do, lse)
    for b in range(2):
        for h in range(Hq):
            got = attention_bwd_rows(q, k, v, do, o, lse, b, h, range(T))
            assert max_abs(got, dq[b, h]) < 1e-10
        for hk in range(Hkv):
            gk, gv = attention_bwd_keys(q, k, v, do, o, lse, b, hk, range(T))
            assert max_abs(gk, dk[b, hk]) < 1e-10
            assert max_abs(gv, dv[b, hk]) < 1e-10


def test_planted_dropped_delta_in_key_form_is_caught():
    q, k, v, do = _rand(1, 2, 1, 30, 64, seed=22)
    o, lse = attention_fwd(q, k, v)
    _, dk, _ = attention_bwd(q, k, v, o, do, lse)
    bad, _ = attention_bwd_keys(q, k, v, do, torch.zeros_like(o), lse, 0, 0, range(30))
    assert max_abs(bad, dk[0, 0]) > 1e-3


# ------------------------------------------------------- seeded workload inputs
def test_workload_inputs_are_reproducible_and_shaped():
    for name in ("C1", "C3"):
        cfg = CONFIGS[name]
        a = make_inputs(cfg, seed=0, batch=1)
        b = make_inputs(cfg, seed=0, batch=1)
        for x, y in zip(a[:4], b[:4]):
            assert torch.equal(x, y)
        q, k, v, do, _ = a
        assert q.shape == (1, cfg.Hq, cfg.T, cfg.D) and k.shape == (1, cfg.Hkv, cfg.T, cfg.D)
        assert q.dtype == cfg.dtype
        rms = q.float().pow(2).mean(-1).sqrt()
        assert (rms - 1).abs().max() < 1e-2  # unit-RMS per head along D (bf16 rounding)


def test_outlier_channels_c4():
    cfg = CONFIGS["C4"]
    q, k, _, _, ch = make_inputs(cfg, seed=0, batch=1)
    assert len(ch) == max(1, round(0.01 * cfg.D)) == 1
    qf = q.float()
    # The outlier channel carries ~8x the RMS of the others, identically in q and k.
    big = qf[..., ch].abs().mean()
    rest = qf[..., [c for c in range(cfg.D) if c not in ch]].abs().mean()
    assert 6 < float(big / rest) < 10


def test_flop_convention():
    cfg = CONFIGS["C2"]
    assert cfg.fwd_flop() == 2.0 * 16 * 12 * 1024 * 1024 * 64
    assert math.isclose(cfg.fwd_flop() / 1e9, 25.77, rel_tol=1e-3)
    assert cfg.bwd_flop() == 2.5 * cfg.fwd_flop()


def test_make_custom_matches_reference_test_shapes():
    q, k, v, do = make_custom(2, 8, 2, 500, 128, torch.bfloat16, seed=0)
    assert q.shape == (2, 8, 500, 128) and k.shape == (2, 2, 500, 128)
    assert all(t.is_contiguous() and t.dtype == torch.bfloat16 for t in (q, k, v, do))


def _block_diag_dense(q, k, v, cu):
    """Dense fp64 attention over all packed rows with an explicit block-diagonal causal
    mask (row i may see column j iff both lie in one sequence and j <= i)."""
    Hq, total, D = q.shape
    G = Hq // k.shape[0]
    kk, vv = k.double().repeat_interleave(G, 0), v.double().repeat_interleave(G, 0)
    seq = torch.zeros(total, dtype=torch.long)
    for s, (c0, c1) in enumerate(zip(cu[:-1], cu[1:])):
        seq[c0:c1] = s
    i = torch.arange(total)
    allowed = (seq[:, None] == seq[None, :]) & (i[None, :] <= i[:, None])
    s_ = q.double() @ kk.transpose(-1, -2) / math.sqrt(D)
    s_ = s_.masked_fill(~allowed, float("-inf"))
    return torch.softmax(s_, -1) @ vv, torch.logsumexp(s_, -1)


def test_varlen_reference_is_block_diagonal_causal_attention():
    g = torch.Generator().manual_seed(3)
    cu = [0, 1, 9, 9, 40, 64]  # includes an empty sequence and a length-1 sequence
    q = torch.randn(4, 64, 64, generator=g)
    k = torch.randn(2, 64, 64, generator=g)
    v = torch.randn(2, 64, 64, generator=g)
    do = torch.randn(4, 64, 64, generator=g)
    o, lse, dq, dk, dv = varlen_reference(q, k, v, do, cu, dtype=torch.float64)
    o_d, lse_d = _block_diag_dense(q, k, v, cu)
    torch.testing.assert_close(o, o_d, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(lse, lse_d, rtol=1e-10, atol=1e-10)
    # gradients of the dense formulation through autograd
    qr, kr, vr = (t.double().requires_grad_() for t in (q, k, v))
    o_a, _ = _block_diag_dense(qr, kr, vr, cu)
    o_a.backward(do.double())
    for a, b in ((dq, qr.grad), (dk, kr.grad), (dv, vr.grad)):
        torch.testing.assert_close(a, b, rtol=1e-9, atol=1e-9)


def test_planted_mask_leak_across_sequences_is_caught():
    """Running the packed rows as one causal sequence (the mistake of ignoring
    cu_seqlens) differs from the block-diagonal reference."""
    g = torch.Generator().manual_seed(4)
    cu = [0, 20, 50]
    q, k, v = (torch.randn(2, 50, 64, generator=g) for _ in range(3))
    o, *_ = varlen_reference(q, k, v, torch.zeros_like(q), cu, dtype=torch.float64)
    leak, _ = attention_fwd(q[None], k[None], v[None])
    assert (o[:, 20:] - leak[0, :, 20:]).abs().max() > 1e-3
    torch.testing.assert_close(o[:, :20], leak[0, :, :20].to(o.dtype), rtol=1e-10, atol=1e-10)


def test_decode_reference_is_last_rows_of_causal_attention():
    """Decode with the cache holding a sequence's K/V equals the last Tq rows of full
    causal attention over that sequence (per batch, with per-batch lengths)."""
    from oracle.eager_attention import decode_reference

    g = torch.Generator().manual_seed(5)
    B, Hq, Hkv, D, Lmax, Tq = 3, 4, 2, 64, 40, 3
    lens = [40, 17, 3]
    kc = torch.randn(B, Hkv, Lmax, D, generator=g, dtype=torch.float64)
    vc = torch.randn(B, Hkv, Lmax, D, generator=g, dtype=torch.float64)
    qfull = torch.randn(B, Hq, Lmax, D, generator=g, dtype=torch.float64)
    q = torch.stack([qfull[b, :, lens[b] - Tq:lens[b]] for b in range(B)])
    o, lse = decode_reference(q, kc, vc, lens)
    for b in range(B):
        L = lens[b]
        of, lf = attention_fwd(qfull[b:b + 1, :, :L], kc[b:b + 1, :, :L], vc[b:b + 1, :, :L])
        torch.testing.assert_close(o[b], of[0, :, L - Tq:L], rtol=1e-10, atol=1e-10)
        torch.testing.assert_close(lse[b], lf[0, :, L - Tq:L], rtol=1e-10, atol=1e-10)


def test_decode_reference_rows_without_keys():
    from oracle.eager_attention import decode_reference

    q = torch.randn(1, 2, 4, 64, dtype=torch.float64)
    kc = torch.randn(1, 1, 8, 64, dtype=torch.float64)
    o, lse = decode_reference(q, kc, kc, [2])  # rows 0, 1 sit at positions -2, -1
    assert torch.all(o[0, :, :2] == 0) and torch.all(torch.isinf(lse[0, :, :2]))
    assert torch.isfinite(lse[0, :, 2:]).all()
