"""CPU tests of the C ABI (libttfa.so) and the host-side op surface.

No compute call runs here: the library is loaded, its exports are checked against
include/ttfa.h, and every argument-validation path is exercised (validation returns
before any HIP call, include/ttfa.h).  The Python side is checked for the reference's
op names, schemas, fake shapes, autograd registration and loud failure modes
(kernels/flash_attn.py:220-327; model.py:92-98; pretrain.py:226-231).
"""

import ctypes
import math
import re
from pathlib import Path

import pytest
import torch

from tinytrain_amd import _lib
from tinytrain_amd.attention import ATTN_IMPLS, causal_attention, validate_attn_impl
from tinytrain_amd.kernels import flash_attn as fa

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "ttfa.h"

needs_lib = pytest.mark.skipif(not _lib.LIB_PATH.exists(),
                               reason="libttfa.so not built (python -m tinytrain_amd.build)")


def _declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?(?:\w+\s+)*\w+\s*\*?\s*(ttfa_\w+)\s*\(", text,
                                 flags=re.M)))


def test_header_declares_the_python_binding():
    assert _declared_functions() == sorted(_lib.EXPORTED)


@needs_lib
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} declared in ttfa.h but not exported"
    assert _lib.load().ttfa_abi_version() == _lib.ABI_VERSION


@needs_lib
@needs_lib
def test_d128_kernel_choice_is_a_rule_on_the_shape():
    # The 256-row D = 128 kernels run where their pairs number at least 256 and T is long
    # enough (dQ pass: T > 1792, forward: T > 3840); no HIP call, so it runs here.
    cases = {
        (4, 16, 4096): (True, True),      # C4
        (1, 16, 16384): (True, True),     # C5
        (32, 8, 512): (False, False),     # REF112M, the reference model's shape
        (1, 64, 2000): (False, True),     # 64 heads x 4 pairs = 256: exactly one per CU
        (1, 64, 1792): (False, False),    # 7 row tiles of 256: below the dQ threshold
        (1, 63, 2000): (False, False),    # 252 pairs: fewer than 256
        (1, 32, 4000): (True, True),      # 32 x 8 pairs
        (1, 31, 4000): (False, False),    # 31 x 8 = 248 pairs
    }
    for (B, Hq, T), want in cases.items():
        assert _lib.d128_wide(B, Hq, T) == want, (B, Hq, T)
    lib = _lib.load()
    f, d = ctypes.c_int(), ctypes.c_int()
    assert lib.ttfa_d128_wide(0, 8, 512, ctypes.byref(f), ctypes.byref(d)) == _lib.E_SEQ
    assert lib.ttfa_d128_wide(1, 8, 0, ctypes.byref(f), ctypes.byref(d)) == _lib.E_SEQ
    assert lib.ttfa_d128_wide(1, 8, 512, None, ctypes.byref(d)) == _lib.E_NULL


@pytest.mark.parametrize("code", [-1, -2, -3, -4, -5, -6, -7, -8, -9])
def test_strerror_names_validation_codes(code):
    msg = _lib.strerror(code)
    assert msg.startswith("ttfa:") and "unknown" not in msg


# Fake, 16-byte aligned, non-null device addresses: every call below fails validation
# and returns before touching them or the HIP runtime.
P = [0x100000 + 0x1000 * i for i in range(10)]
OK = dict(B=1, Hq=4, Hkv=2, T=128, D=64, dtype=_lib.TTFA_BF16, scale=0.125)


def _fwd(ptrs=None, **kw):
    a = {**OK, **kw}
    p = P[:5] if ptrs is None else ptrs
    return _lib.load().ttfa_fwd(*p, a["B"], a["Hq"], a["Hkv"], a["T"], a["D"], a["dtype"],
                                a["scale"], None)


def _bwd(ptrs=None, **kw):
    a = {**OK, **kw}
    p = P[:10] if ptrs is None else ptrs
    return _lib.load().ttfa_bwd(*p, a["B"], a["Hq"], a["Hkv"], a["T"], a["D"], a["dtype"],
                                a["scale"], None)


def _bwd_dq(ptrs=None, **kw):
    a = {**OK, **kw}
    p = P[:8] if ptrs is None else ptrs
    return _lib.load().ttfa_bwd_dq(*p, a["B"], a["Hq"], a["Hkv"], a["T"], a["D"], a["dtype"],
                                   a["scale"], None)


def _bwd_dkdv(ptrs=None, **kw):
    a = {**OK, **kw}
    p = P[:8] if ptrs is None else ptrs
    return _lib.load().ttfa_bwd_dkdv(*p, a["B"], a["Hq"], a["Hkv"], a["T"], a["D"],
                                     a["dtype"], a["scale"], None)


CASES = [
    (dict(D=96), _lib.E_HEAD_DIM),
    (dict(D=32), _lib.E_HEAD_DIM),
    (dict(Hq=3, Hkv=2), _lib.E_GROUP),
    (dict(Hkv=0), _lib.E_GROUP),
    (dict(Hq=0), _lib.E_GROUP),
    (dict(T=0), _lib.E_SEQ),
    (dict(B=0), _lib.E_SEQ),
    (dict(T=1 << 24), _lib.E_SEQ),          # one head's bytes exceed the 2 GiB window
    # fp32: one workgroup per 16-row block of every query and KV head, 2^31 of them
    (dict(dtype=1, D=64, B=1 << 14, Hq=1, Hkv=1, T=1 << 20), _lib.E_SEQ),
    (dict(dtype=2), _lib.E_DTYPE),
    (dict(dtype=-1), _lib.E_DTYPE),
    (dict(scale=0.0), _lib.E_SCALE),
    (dict(scale=-0.1), _lib.E_SCALE),
    (dict(scale=math.inf), _lib.E_SCALE),
    (dict(scale=math.nan), _lib.E_SCALE),
]


@needs_lib
@pytest.mark.parametrize("entry", [_fwd, _bwd, _bwd_dq, _bwd_dkdv])
@pytest.mark.parametrize("kw, code", CASES)
def test_argument_errors_return_codes(entry, kw, code):
    assert entry(**kw) == code


@needs_lib
@pytest.mark.parametrize("entry, n", [(_fwd, 5), (_bwd, 10), (_bwd_dq, 8), (_bwd_dkdv, 8)])
def test_null_and_misaligned_pointers(entry, n):
    for i in range(n):
        ptrs = list(P[:n])
        ptrs[i] = None
        assert entry(ptrs=ptrs) == _lib.E_NULL
        ptrs[i] = P[i] + 8
        assert entry(ptrs=ptrs) == _lib.E_ALIGN


@needs_lib
def test_check_raises_with_message():
    with pytest.raises(_lib.TTFAError, match="head dim"):
        _lib.check(_fwd(D=80))


# ------------------------------------------------------------ Python op surface
def test_custom_ops_registered_with_reference_schemas():
    fwd = torch.ops.tinytrain.flash_attn_fwd.default
    bwd = torch.ops.tinytrain.flash_attn_bwd.default
    assert [a.name for a in fwd._schema.arguments] == ["q", "k", "v"]
    assert len(fwd._schema.returns) == 2
    assert [a.name for a in bwd._schema.arguments] == ["q", "k", "v", "o", "do", "M"]
    assert len(bwd._schema.returns) == 3


def test_fake_impls_and_autograd_under_fake_mode():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        q = torch.empty(2, 8, 64, 128, dtype=torch.bfloat16, requires_grad=True)
        k = torch.empty(2, 2, 64, 128, dtype=torch.bfloat16, requires_grad=True)
        v = torch.empty(2, 2, 64, 128, dtype=torch.bfloat16, requires_grad=True)
        o, M = fa.flash_attn_fwd(q, k, v)
        assert o.shape == q.shape and o.dtype == q.dtype
        assert M.shape == (2, 8, 64) and M.dtype == torch.float32
        o.float().sum().backward()
        assert q.grad.shape == q.shape and k.grad.shape == k.shape and v.grad.shape == v.shape


def test_compile_fullgraph_traces_one_opaque_node():
    # Dynamo traces through the fake impl with fullgraph=True (a graph break would raise
    # during tracing); the captured graph holds the custom op, never the ctypes call.
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)
        return gm.forward

    def f(q, k, v):
        return fa.flash_attn(q, k, v) * 2

    q = torch.randn(1, 4, 16, 64)
    k = torch.randn(1, 2, 16, 64)
    cf = torch.compile(f, backend=backend, fullgraph=True)
    with pytest.raises(fa.FlashAttnInputError, match="ROCm GPU"):
        cf(q, k, k)  # traced, then the real op rejects CPU tensors loudly
    assert len(graphs) == 1
    assert "tinytrain.flash_attn_fwd" in str(graphs[0].graph)


def _t(*s, dtype=torch.bfloat16):
    return torch.zeros(*s, dtype=dtype)


@pytest.mark.parametrize("q, k, v, match", [
    (_t(1, 4, 8, 64).transpose(2, 3), _t(1, 4, 64, 8), _t(1, 4, 64, 8), "contiguous"),
    (_t(4, 8, 64), _t(4, 8, 64), _t(4, 8, 64), "4-D"),
    (_t(1, 4, 8, 64), _t(1, 3, 8, 64), _t(1, 3, 8, 64), "multiple"),
    (_t(1, 4, 8, 96), _t(1, 4, 8, 96), _t(1, 4, 8, 96), "head dim"),
    (_t(1, 4, 8, 64), _t(1, 4, 8, 64, dtype=torch.float16), _t(1, 4, 8, 64), "dtype"),
    (_t(1, 4, 8, 64), _t(1, 2, 9, 64), _t(1, 2, 9, 64), "matching"),
    (_t(1, 4, 8, 64), _t(1, 2, 8, 64), _t(1, 2, 8, 64), "ROCm GPU"),
])
def test_forward_rejects_bad_inputs_loudly(q, k, v, match):
    with pytest.raises(fa.FlashAttnInputError, match=match):
        fa._forward(q, k, v)


def test_non_contiguous_is_also_an_assertion_error():
    # The reference asserts contiguity (kernels/flash_attn.py:221-223).
    q = _t(1, 4, 64, 8).transpose(2, 3)
    with pytest.raises(AssertionError):
        fa._forward(q, _t(1, 4, 8, 64), _t(1, 4, 8, 64))


def test_attn_impl_switch_validates_names():
    assert ATTN_IMPLS == ("sdpa", "hip")
    assert validate_attn_impl("hip") == "hip"
    for bad in ("triton", "flash", "", "HIP"):
        with pytest.raises(ValueError):
            validate_attn_impl(bad)


def test_sdpa_branch_is_the_eager_path():
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 4, 12, 64, generator=g)
    k = torch.randn(1, 2, 12, 64, generator=g)
    v = torch.randn(1, 2, 12, 64, generator=g)
    a = causal_attention(q, k, v, "sdpa", enable_gqa=False)
    b = causal_attention(q, k, v, "sdpa", enable_gqa=True)
    assert torch.allclose(a, b, atol=1e-6)


def test_hip_switch_on_cpu_fails_loudly():
    q = torch.randn(1, 2, 8, 64)
    with pytest.raises(fa.FlashAttnInputError):
        causal_attention(q, q, q, "hip")


def test_reference_import_path_reexports_the_same_ops():
    """`from kernels.flash_attn import ...` (model.py:6, tests/test_flash_attn.py:4)
    resolves to the same op objects as the package path."""
    from kernels import flash_attn as ref_path

    for name in ("_forward", "_backward", "flash_attn", "flash_attn_fwd", "flash_attn_bwd"):
        assert getattr(ref_path, name) is getattr(fa, name)


def test_fused_prologue_needs_one_eps(monkeypatch):
    """The fused q/k prologue takes one eps; with q_norm.eps != k_norm.eps the block runs
    the eager norm lines instead (the fused op is never called)."""
    from tinytrain_amd import attention as att

    def fused_must_not_run(*a, **k):
        raise AssertionError("fused prologue used with two different eps")

    monkeypatch.setattr(att, "qk_norm_rope", fused_must_not_run)
    monkeypatch.setattr(att, "causal_attention",
                        lambda q, k, v, impl, gqa: causal_attention(q, k, v, "sdpa", gqa))
    blk = att.Attention(64, 4, 2, 16, eps=1e-6)
    blk.attn_impl, blk.fused_prologue = "hip", True
    blk.k_norm.eps = 1e-5
    cos, sin = att.precompute_rope(16, 8, 10000.0)
    out = blk(torch.randn(1, 8, 64), cos, sin)
    assert out.shape == (1, 8, 64)


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libttfa.so")
    with pytest.raises(_lib.LibraryNotBuilt, match="missing"):
        _lib.load()


# ------------------------------------------------------------------ varlen entry points
VL = dict(n_seq=3, total=300, max_seqlen=128, Hq=4, Hkv=2, D=64, dtype=_lib.TTFA_BF16,
          scale=0.125)
CU = 0x300000  # fake, 4-byte aligned device address of cu_seqlens


def _vl_fwd(ptrs=None, cu=CU, **kw):
    a = {**VL, **kw}
    p = list(P[:5]) if ptrs is None else ptrs
    return _lib.load().ttfa_varlen_fwd(*p, cu, a["n_seq"], a["total"], a["max_seqlen"], a["Hq"],
                                       a["Hkv"], a["D"], a["dtype"], a["scale"], None)


def _vl_bwd(ptrs=None, cu=CU, **kw):
    a = {**VL, **kw}
    p = list(P[:10]) if ptrs is None else ptrs
    return _lib.load().ttfa_varlen_bwd(*p, cu, a["n_seq"], a["total"], a["max_seqlen"], a["Hq"],
                                       a["Hkv"], a["D"], a["dtype"], a["scale"], None)


@needs_lib
@pytest.mark.parametrize("call", [_vl_fwd, _vl_bwd])
@pytest.mark.parametrize("kw,code", [
    (dict(dtype=_lib.TTFA_F32), _lib.E_DTYPE), (dict(D=96), _lib.E_HEAD_DIM),
    (dict(Hq=3), _lib.E_GROUP), (dict(n_seq=0), _lib.E_SEQ), (dict(total=0), _lib.E_SEQ),
    (dict(max_seqlen=0), _lib.E_SEQ), (dict(max_seqlen=1 << 24, D=128), _lib.E_SEQ),
    (dict(scale=0.0), _lib.E_SCALE),
])
def test_varlen_abi_validation(call, kw, code):
    assert call(**kw) == code


@needs_lib
@pytest.mark.parametrize("call,n", [(_vl_fwd, 5), (_vl_bwd, 10)])
def test_varlen_abi_pointer_checks(call, n):
    assert call(cu=None) == _lib.E_NULL
    assert call(cu=CU + 2) == _lib.E_ALIGN
    for i in range(n):
        p = list(P[:n])
        p[i] = None
        assert call(p) == _lib.E_NULL
        p = list(P[:n])
        p[i] = P[i] + 8
        assert call(p) == _lib.E_ALIGN


@pytest.mark.parametrize("bad,msg", [("rank", "3-D"), ("dtype", "bfloat16"),
                                     ("cu_dtype", "int32"), ("group", "multiple"),
                                     ("cpu", "ROCm GPU")])
def test_varlen_input_errors(bad, msg):
    q = torch.zeros(4, 300, 64, dtype=torch.bfloat16)
    k = torch.zeros(2, 300, 64, dtype=torch.bfloat16)
    cu = torch.tensor([0, 100, 300], dtype=torch.int32)
    if bad == "rank":
        q = q[None]
    elif bad == "dtype":
        q = q.float()
    elif bad == "cu_dtype":
        cu = cu.long()
    elif bad == "group":
        q = torch.zeros(3, 300, 64, dtype=torch.bfloat16)
    with pytest.raises(fa.FlashAttnInputError, match=msg):
        fa.flash_attn_varlen(q, k, k, cu, 200)


def test_varlen_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(8, 1000, 128, dtype=torch.bfloat16)
        k = torch.empty(2, 1000, 128, dtype=torch.bfloat16)
        cu = torch.empty(5, dtype=torch.int32)
        o, M = torch.ops.tinytrain.flash_attn_varlen_fwd(q, k, k, cu, 512)
        assert o.shape == q.shape and M.shape == (8, 1000) and M.dtype == torch.float32
        dq, dk, dv = torch.ops.tinytrain.flash_attn_varlen_bwd(q, k, k, o, o, M, cu, 512)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape


# ------------------------------------------------------------------ decode entry points
DC = dict(B=2, Hq=8, Hkv=2, Tq=1, L=1024, D=128, dtype=_lib.TTFA_BF16, scale=0.0884)


def _dec(ptrs=None, lens=CU, **kw):
    a = {**DC, **kw}
    p = list(P[:3]) + [lens] + list(P[3:6]) if ptrs is None else ptrs
    return _lib.load().ttfa_decode_fwd(*p, a["B"], a["Hq"], a["Hkv"], a["Tq"], a["L"], a["D"],
                                       a["dtype"], a["scale"], None)


@needs_lib
@pytest.mark.parametrize("kw,code", [
    (dict(dtype=_lib.TTFA_F32), _lib.E_DTYPE), (dict(D=80), _lib.E_HEAD_DIM),
    (dict(Hq=7), _lib.E_GROUP), (dict(B=0), _lib.E_SEQ), (dict(Tq=0), _lib.E_SEQ),
    (dict(L=0), _lib.E_SEQ), (dict(Tq=9), _lib.E_QROWS), (dict(scale=-1.0), _lib.E_SCALE),
])
def test_decode_abi_validation(kw, code):
    assert _dec(**kw) == code


@needs_lib
def test_decode_abi_pointers_and_workspace():
    assert _dec(lens=None) == _lib.E_NULL
    assert _dec(lens=CU + 1) == _lib.E_ALIGN
    for i in (0, 1, 2, 4, 5, 6):
        p = list(P[:3]) + [CU] + list(P[3:6])
        p[i] = None
        assert _dec(p) == _lib.E_NULL
    lib = _lib.load()
    n = lib.ttfa_decode_workspace_bytes(2, 8, 2, 1, 1024, 128)
    assert n > 0 and n % (4 * (128 + 2)) == 0
    assert lib.ttfa_decode_workspace_bytes(2, 8, 2, 9, 1024, 128) == -1
    assert _lib.strerror(_lib.E_QROWS).startswith("ttfa:")


def test_decode_input_errors_and_fake():
    from torch._subclasses.fake_tensor import FakeTensorMode

    from tinytrain_amd.kernels.decode import flash_attn_decode

    q = torch.zeros(2, 8, 1, 64, dtype=torch.bfloat16)
    kc = torch.zeros(2, 2, 100, 64, dtype=torch.bfloat16)
    lens = torch.tensor([100, 50], dtype=torch.int32)
    with pytest.raises(fa.FlashAttnInputError, match="32 query rows"):
        flash_attn_decode(torch.zeros(2, 8, 9, 64, dtype=torch.bfloat16), kc, kc, lens)
    with pytest.raises(fa.FlashAttnInputError, match="int32"):
        flash_attn_decode(q, kc, kc, lens.long())
    with pytest.raises(fa.FlashAttnInputError, match="ROCm GPU"):
        flash_attn_decode(q, kc, kc, lens)
    with FakeTensorMode():
        qf = torch.empty(2, 8, 1, 64, dtype=torch.bfloat16)
        kf = torch.empty(2, 2, 100, 64, dtype=torch.bfloat16)
        lf = torch.empty(2, dtype=torch.int32)
        o, lse = torch.ops.tinytrain.flash_attn_decode(qf, kf, kf, lf)
        assert o.shape == qf.shape and lse.shape == (2, 8, 1) and lse.dtype == torch.float32
