"""CPU tests of the fused attention prologue: the oracle's pins and the host surface.

The oracle (oracle/qk_prologue.py) restates model.py:24-56 / :83-93 of the reference;
here it is checked against a library routine (torch's rms_norm), closed forms, the
rotation structure of RoPE, finite differences, and planted mistakes.  The C ABI's
validation paths and the Python op surface are checked without a GPU (validation
returns before any HIP call).
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import qk_prologue as oq
from tinytrain_amd import _lib
from tinytrain_amd.kernels import qk_prologue as qp

needs_lib = pytest.mark.skipif(not _lib.LIB_PATH.exists(), reason="libttfa.so not built")


def _inputs(B=2, T=9, Hq=4, Hkv=2, D=64, dtype=torch.float64, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, Hq, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, T, Hkv, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, T, Hkv, D, generator=g, dtype=torch.float64)
    wq = 1 + 0.1 * torch.randn(D, generator=g, dtype=torch.float64)
    wk = 1 + 0.1 * torch.randn(D, generator=g, dtype=torch.float64)
    cos, sin = oq.rope_tables(D, 64, 1e6, torch.float64)
    return [t.to(dtype) for t in (q, k, v)] + [wq, wk, cos, sin]


# ---------------------------------------------------------------- oracle pins
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-6), (torch.float64, 1e-12)])
def test_rms_norm_matches_library(dtype, tol):
    x = torch.randn(5, 7, 64, dtype=dtype)
    w = torch.randn(64, dtype=dtype)
    ref = F.rms_norm(x, (64,), w, eps=1e-6)
    torch.testing.assert_close(oq.rms_norm(x, w, 1e-6), ref, rtol=tol, atol=tol)


def test_rms_norm_constant_rows_closed_form():
    eps = 1e-6
    c = torch.tensor([-3.0, -0.5, 0.25, 2.0], dtype=torch.float64)
    x = c[:, None].expand(4, 128).clone()
    w = torch.linspace(0.5, 1.5, 128, dtype=torch.float64)
    want = w[None, :] * torch.sign(c)[:, None] / torch.sqrt(1 + eps / c[:, None] ** 2)
    torch.testing.assert_close(oq.rms_norm(x, w, eps), want, rtol=1e-12, atol=1e-12)


def test_rope_position_zero_is_identity():
    x = torch.randn(3, 1, 64, dtype=torch.float64)
    cos, sin = oq.rope_tables(64, 4, 1e6, torch.float64)
    torch.testing.assert_close(oq.apply_rope(x, cos[:1], sin[:1]), x, rtol=0, atol=0)


def test_rope_is_a_rotation_of_column_pairs():
    D, T = 64, 16
    x = torch.randn(T, D, dtype=torch.float64)
    cos, sin = oq.rope_tables(D, T, 1e6, torch.float64)
    y = oq.apply_rope(x, cos, sin)
    h = D // 2
    # pair norms preserved
    torch.testing.assert_close(x[:, :h] ** 2 + x[:, h:] ** 2, y[:, :h] ** 2 + y[:, h:] ** 2,
                               rtol=1e-12, atol=1e-12)
    # explicit 2x2 rotation of one pair: (a, b) -> (a cos - b sin, a sin + b cos)
    t, i = 7, 5
    ang = t * 1e6 ** (-(2 * i) / D)
    a, b = x[t, i], x[t, i + h]
    assert math.isclose(float(y[t, i]), float(a * math.cos(ang) - b * math.sin(ang)), abs_tol=1e-12)
    assert math.isclose(float(y[t, i + h]), float(a * math.sin(ang) + b * math.cos(ang)),
                        abs_tol=1e-12)


def test_rope_angles_compose():
    D = 128
    x = torch.randn(4, D, dtype=torch.float64)
    cos, sin = oq.rope_tables(D, 32, 1e6, torch.float64)
    a, b = 5, 11
    twice = oq.apply_rope(oq.apply_rope(x, cos[a], sin[a]), cos[b], sin[b])
    torch.testing.assert_close(twice, oq.apply_rope(x, cos[a + b], sin[a + b]), rtol=1e-10,
                               atol=1e-10)


def test_prologue_layout_and_rstd():
    q, k, v, wq, wk, cos, sin = _inputs()
    qo, ko, vo, rq, rk = oq.qk_prologue(q, k, v, wq, wk, cos, sin)
    assert qo.shape == (2, 4, 9, 64) and ko.shape == (2, 2, 9, 64) and qo.is_contiguous()
    torch.testing.assert_close(vo, v.transpose(1, 2), rtol=0, atol=0)
    torch.testing.assert_close(rq, 1 / torch.sqrt(q.pow(2).mean(-1) + 1e-6), rtol=1e-12, atol=0)
    # row (b, h, t) of the output is RoPE(norm(row (b, t, h))) at position t
    b, h, t = 1, 3, 6
    want = oq.apply_rope(oq.rms_norm(q[b, t, h], wq), cos[t], sin[t])
    torch.testing.assert_close(qo[b, h, t], want, rtol=1e-12, atol=1e-12)


def test_prologue_gradcheck():
    q, k, v, wq, wk, cos, sin = _inputs(B=1, T=3, Hq=2, Hkv=1, D=64)
    ins = [t.clone().requires_grad_() for t in (q, k, v, wq, wk)]

    def f(q, k, v, wq, wk):
        return oq.qk_prologue(q, k, v, wq, wk, cos, sin)[:3]

    assert torch.autograd.gradcheck(f, ins, eps=1e-6, atol=1e-7)


def test_bf16_path_within_rounding_of_fp64():
    q, k, v, wq, wk, cos, sin = _inputs(D=128)
    exact = oq.qk_prologue(q, k, v, wq, wk, cos, sin)
    qb, kb, vb = (t.to(torch.bfloat16) for t in (q, k, v))
    bf = oq.qk_prologue(qb, kb, vb, wq.float(), wk.float(), cos.float(), sin.float())
    exact_b = oq.qk_prologue(qb.double(), kb.double(), vb.double(), wq, wk, cos, sin)
    for a, e in zip(bf[:3], exact_b[:3]):
        err = (a.double() - e).abs().max().item()
        assert err <= 3 * 2 ** -8 * max(1.0, e.abs().max().item()), err
    assert exact[0].shape == bf[0].shape


@pytest.mark.parametrize("mistake", ["rot_sign", "norm_dim", "no_eps_sqrt"])
def test_planted_mistakes_fail_the_pins(mistake):
    """Plausible mistakes in a restatement are caught by the checks above."""
    x = torch.randn(6, 64, dtype=torch.float64)
    w = torch.ones(64, dtype=torch.float64)
    cos, sin = oq.rope_tables(64, 8, 1e6, torch.float64)
    if mistake == "rot_sign":  # cat(x2, -x1) instead of cat(-x2, x1)
        x1, x2 = x.chunk(2, dim=-1)
        bad = x * cos[3] + torch.cat([x2, -x1], dim=-1) * sin[3]
        good = oq.apply_rope(x, cos[3], sin[3])
        assert not torch.allclose(bad, good)
        # it is a rotation by -angle: composition with +angle no longer gives angle 2a
        assert not torch.allclose(oq.apply_rope(bad, cos[3], sin[3]), oq.apply_rope(x, cos[6], sin[6]))
    elif mistake == "norm_dim":  # mean over the wrong axis
        bad = w * x * torch.rsqrt(x.pow(2).mean(dim=0, keepdim=True) + 1e-6)
        assert not torch.allclose(bad, F.rms_norm(x, (64,), w, eps=1e-6))
    else:  # rsqrt(mean) + eps instead of rsqrt(mean + eps): visible on constant rows
        c = torch.full((2, 64), 1e-3, dtype=torch.float64)
        bad = w * c * (torch.rsqrt(c.pow(2).mean(-1, keepdim=True)) + 1e-6)
        want = w * torch.sign(c) / torch.sqrt(1 + 1e-6 / c ** 2)
        assert not torch.allclose(bad, want, rtol=1e-6, atol=1e-9)


# ---------------------------------------------------------------- C ABI validation
P = [0x200000 + 0x1000 * i for i in range(17)]
OK = dict(B=1, T=8, Hq=4, Hkv=2, D=64)


def _fwd(ptrs=None, eps=1e-6, **kw):
    a = {**OK, **kw}
    p = list(P[:12]) if ptrs is None else ptrs
    return _lib.load().ttfa_qk_prologue_fwd(*p, a["B"], a["T"], a["Hq"], a["Hkv"], a["D"], eps, None)


def _bwd(ptrs=None, **kw):
    a = {**OK, **kw}
    p = list(P[:17]) if ptrs is None else ptrs
    return _lib.load().ttfa_qk_prologue_bwd(*p, a["B"], a["T"], a["Hq"], a["Hkv"], a["D"], None)


@needs_lib
@pytest.mark.parametrize("call", [_fwd, _bwd])
@pytest.mark.parametrize("kw,code", [
    (dict(D=96), _lib.E_HEAD_DIM), (dict(D=32), _lib.E_HEAD_DIM),
    (dict(Hq=3, Hkv=2), _lib.E_GROUP), (dict(Hkv=0), _lib.E_GROUP),
    (dict(B=0), _lib.E_SEQ), (dict(T=0), _lib.E_SEQ),
])
def test_abi_rejects_bad_shapes(call, kw, code):
    assert call(**kw) == code


@needs_lib
@pytest.mark.parametrize("call,n", [(_fwd, 12), (_bwd, 17)])
def test_abi_rejects_null_and_misaligned(call, n):
    for i in range(n):
        p = list(P[:n])
        p[i] = None
        assert call(p) == _lib.E_NULL
        p = list(P[:n])
        p[i] = P[i] + 4
        assert call(p) == _lib.E_ALIGN


@needs_lib
@pytest.mark.parametrize("eps", [-1e-6, 1.0, float("nan")])
def test_abi_rejects_bad_eps(eps):
    assert _fwd(eps=eps) == _lib.E_EPS


@needs_lib
def test_workspace_bytes():
    lib = _lib.load()
    # backward at D=128: 16 rows in flight x 8 rounds = 128 rows per workgroup, one fp32
    # partial of D values per q or k workgroup
    B, T, Hq, Hkv, D = 2, 100, 8, 2, 128
    nq = -(-B * T * Hq // 128)
    nk = -(-B * T * Hkv // 128)
    assert lib.ttfa_qk_prologue_workspace_bytes(B, T, Hq, Hkv, D) == (nq + nk) * D * 4
    assert lib.ttfa_qk_prologue_workspace_bytes(B, T, Hq, Hkv, 96) == -1


# ---------------------------------------------------------------- Python op surface
def test_ops_registered_with_schemas():
    fwd = torch.ops.tinytrain.qk_norm_rope_fwd.default
    bwd = torch.ops.tinytrain.qk_norm_rope_bwd.default
    assert len(fwd._schema.arguments) == 8 and len(fwd._schema.returns) == 5
    assert len(bwd._schema.arguments) == 11 and len(bwd._schema.returns) == 5


def test_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(2, 16, 8, 128, dtype=torch.bfloat16)
        k = torch.empty(2, 16, 2, 128, dtype=torch.bfloat16)
        w = torch.empty(128)
        cs = torch.empty(32, 128)
        out = torch.ops.tinytrain.qk_norm_rope_fwd(q, k, k, w, w, cs, cs, 1e-6)
        assert [tuple(t.shape) for t in out] == [(2, 8, 16, 128), (2, 2, 16, 128),
                                                 (2, 2, 16, 128), (2, 16, 8), (2, 16, 2)]
        assert out[0].dtype == torch.bfloat16 and out[3].dtype == torch.float32


@pytest.mark.parametrize("bad,msg", [("dtype", "bfloat16"), ("contig", "contiguous"),
                                     ("cpu", "ROCm GPU"), ("weight", "weight"),
                                     ("table", "tables"), ("D", "head dim")])
def test_input_errors_are_loud(bad, msg):
    q, k, v, wq, wk, cos, sin = _inputs(dtype=torch.bfloat16)
    wq, wk, cos, sin = wq.float(), wk.float(), cos.float(), sin.float()
    if bad == "dtype":
        q = q.float()
    elif bad == "contig":
        q = q.transpose(1, 2).contiguous().transpose(1, 2)
    elif bad == "weight":
        wq = wq[:32]
    elif bad == "table":
        cos = cos[:4]
    elif bad == "D":
        q, k, v = q[..., :32], k[..., :32], v[..., :32]
    with pytest.raises(qp.QKPrologueInputError, match=msg):
        qp.qk_norm_rope(q, k, v, wq, wk, cos, sin)
