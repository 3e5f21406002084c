"""GPU parity tests of the fused attention prologue (q/k RMSNorm + RoPE + layout).

The HIP op is compared with the CPU oracle (oracle/qk_prologue.py, the reference's
model.py:24-56 / :83-93 expressions) on the same seeded bf16 inputs:

* forward outputs: within one bf16 rounding step (the only freedom is the fp32
  summation order of mean(x^2)), and at least 99% of elements bit-identical; v is an
  exact copy; rstd within 1e-6 relative;
* backward: the gradients of the fp64 restatement evaluated on the same bf16 inputs,
  each bf16 input gradient within one bf16 ulp (2^-8 relative, + 1e-4) of the exact
  value, the fp32 norm-weight gradients within 1e-3 of the largest element;
* bitwise determinism, the torch.library op checks, and the Attention block with the
  fused prologue against the same block's eager prologue (both on the HIP attention).
"""

import pytest
import torch

from helpers import announce
from oracle import qk_prologue as oq
from tinytrain_amd.attention import Attention
from tinytrain_amd.kernels.qk_prologue import qk_norm_rope, qk_norm_rope_bwd, qk_norm_rope_fwd

pytestmark = pytest.mark.gpu

DEV = "cuda"
SHAPES = [
    (32, 512, 8, 2, 128),  # the reference model's attention inputs (B, T, Hq, Hkv, D)
    (2, 37, 4, 4, 64),     # ragged T, MHA, D=64
    (3, 1, 12, 4, 64),     # T=1
    (1, 129, 16, 8, 128),  # rows not a multiple of a workgroup's rows
]


def _inputs(B, T, Hq, Hkv, D, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, Hq, D, generator=g).mul(3).to(torch.bfloat16)
    k = torch.randn(B, T, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, T, Hkv, D, generator=g).to(torch.bfloat16)
    wq = 1 + 0.2 * torch.randn(D, generator=g)
    wk = 1 + 0.2 * torch.randn(D, generator=g)
    cos, sin = oq.rope_tables(D, max(T, 8), 1e6, torch.float32)
    return q, k, v, wq, wk, cos, sin


def _dev(*ts):
    return [t.to(DEV) for t in ts]


def _ulp_ok(got, want, frac_exact=0.99):
    """Every element within two bf16 steps at its row's scale (a one-ulp flip of a
    normalised value, from the fp32 summation order of mean(x^2), moves a RoPE product
    by one ulp of the product, and the sum of the two products can be smaller than
    either), and most elements bit-identical."""
    g, w = got.float().cpu(), want.float()
    row = torch.clamp(w.abs().amax(dim=-1, keepdim=True), min=1.0)
    step = row * 2 ** -6  # two bf16 ulps at the row's largest magnitude
    assert bool(((g - w).abs() <= step).all()), f"max|err| {(g - w).abs().max().item():.3e}"
    exact = (g == w).float().mean().item()
    assert exact >= frac_exact, f"only {exact:.4f} of elements bit-identical"
    return exact


@pytest.mark.parametrize("B,T,Hq,Hkv,D", SHAPES)
def test_forward_matches_oracle(B, T, Hq, Hkv, D):
    announce(f"qk prologue fwd B={B} T={T} Hq={Hq} Hkv={Hkv} D={D}")
    q, k, v, wq, wk, cos, sin = _inputs(B, T, Hq, Hkv, D)
    want = oq.qk_prologue(q, k, v, wq, wk, cos, sin)
    got = qk_norm_rope_fwd(*_dev(q, k, v, wq, wk, cos, sin), 1e-6)
    torch.cuda.synchronize()
    _ulp_ok(got[0], want[0])
    _ulp_ok(got[1], want[1])
    assert torch.equal(got[2].cpu(), want[2])
    for r, rw in ((got[3], want[3]), (got[4], want[4])):
        torch.testing.assert_close(r.cpu(), rw, rtol=1e-6, atol=0)
    assert got[0].shape == (B, Hq, T, D) and got[0].is_contiguous()


@pytest.mark.parametrize("B,T,Hq,Hkv,D", SHAPES)
def test_backward_matches_fp64_gradients(B, T, Hq, Hkv, D):
    announce(f"qk prologue bwd B={B} T={T} Hq={Hq} Hkv={Hkv} D={D}")
    q, k, v, wq, wk, cos, sin = _inputs(B, T, Hq, Hkv, D, seed=1)
    g = torch.Generator().manual_seed(2)
    gq = torch.randn(B, Hq, T, D, generator=g).to(torch.bfloat16)
    gk = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    gv = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    # fp64 restatement on the same bf16 inputs; the tables enter as apply_rope uses
    # them, rounded to bf16 (model.py:52-53), which fixes the RoPE Jacobian
    ins = [t.double().requires_grad_() for t in (q, k, v, wq, wk)]
    cb, sb = (t.to(torch.bfloat16).double() for t in (cos, sin))
    outs = oq.qk_prologue(*ins, cb, sb)
    torch.autograd.backward(outs[:3], [gq.double(), gk.double(), gv.double()])
    want = [t.grad for t in ins]
    qd, kd, vd, wqd, wkd, cd, sd = _dev(q, k, v, wq, wk, cos, sin)
    _, _, _, rq, rk = qk_norm_rope_fwd(qd, kd, vd, wqd, wkd, cd, sd, 1e-6)
    got = qk_norm_rope_bwd(*_dev(gq, gk, gv), qd, kd, wqd, wkd, cd, sd, rq, rk)
    torch.cuda.synchronize()
    for name, a, b in zip(("dq_raw", "dk_raw", "dv_raw"), got[:3], want[:3]):
        # the gradient is evaluated in fp32 and rounded once to bf16: within one bf16 ulp
        # (2^-8 relative) of the exact value, plus a small absolute floor for fp32 error
        err = (a.cpu().double() - b).abs()
        bound = b.abs() * 2 ** -8 + 1e-4
        assert bool((err <= bound).all()), f"{name}: max|err| {err.max().item():.3e}, " \
            f"worst ratio {(err / bound).max().item():.2f}"
    for name, a, b in zip(("dwq", "dwk"), got[3:], want[3:]):
        err = (a.cpu().double() - b).abs().max().item()
        assert err <= 1e-3 * max(1.0, b.abs().max().item()), f"{name}: max|err| {err:.3e}"


def test_backward_deterministic():
    announce("qk prologue bwd determinism")
    B, T, Hq, Hkv, D = 8, 256, 8, 2, 128
    q, k, v, wq, wk, cos, sin = _dev(*_inputs(B, T, Hq, Hkv, D))
    _, _, _, rq, rk = qk_norm_rope_fwd(q, k, v, wq, wk, cos, sin, 1e-6)
    gq = torch.randn(B, Hq, T, D, device=DEV).to(torch.bfloat16)
    gk = torch.randn(B, Hkv, T, D, device=DEV).to(torch.bfloat16)
    a = qk_norm_rope_bwd(gq, gk, gk, q, k, wq, wk, cos, sin, rq, rk)
    b = qk_norm_rope_bwd(gq, gk, gk, q, k, wq, wk, cos, sin, rq, rk)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_opcheck():
    announce("qk prologue opcheck")
    q, k, v, wq, wk, cos, sin = _dev(*_inputs(2, 16, 4, 2, 64))
    torch.library.opcheck(qk_norm_rope_fwd, (q, k, v, wq, wk, cos, sin, 1e-6),
                          test_utils=("test_schema", "test_faketensor"))
    _, _, _, rq, rk = qk_norm_rope_fwd(q, k, v, wq, wk, cos, sin, 1e-6)
    gq = torch.randn(2, 4, 16, 64, device=DEV).to(torch.bfloat16)
    gk = torch.randn(2, 2, 16, 64, device=DEV).to(torch.bfloat16)
    torch.library.opcheck(qk_norm_rope_bwd, (gq, gk, gk, q, k, wq, wk, cos, sin, rq, rk),
                          test_utils=("test_schema", "test_faketensor"))


def test_attention_block_fused_vs_eager_prologue():
    """Attention(attn_impl="hip") with and without the fused prologue: same output within
    bf16 rounding, same parameter gradients within the attention tolerance."""
    announce("attention block fused prologue vs eager prologue")
    torch.manual_seed(0)
    hidden, H, Hkv, dh, B, T = 256, 8, 2, 64, 4, 128
    blk = Attention(hidden, H, Hkv, dh).to(DEV)
    with torch.no_grad():
        blk.q_norm.weight.add_(0.1 * torch.randn(dh, device=DEV))
        blk.k_norm.weight.add_(0.1 * torch.randn(dh, device=DEV))
    blk.attn_impl = "hip"
    cos, sin = oq.rope_tables(dh, T, 1e6, torch.float32)
    cos, sin = cos.to(DEV), sin.to(DEV)
    x = torch.randn(B, T, hidden, device=DEV)
    res = []
    for fused in (False, True):
        blk.fused_prologue = fused
        blk.zero_grad()
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            y = blk(x, cos, sin)
        y.float().square().mean().backward()
        res.append((y.detach().float(), {n: p.grad.clone() for n, p in blk.named_parameters()}))
    (y0, g0), (y1, g1) = res
    assert (y0 - y1).abs().max().item() <= 2e-2
    for n in g0:
        scale = max(1.0, g0[n].abs().max().item())
        err = (g0[n] - g1[n]).abs().max().item()
        assert err <= 2e-2 * scale, f"grad {n}: max|err| {err:.3e}"


def test_compile_fullgraph_with_fused_prologue():
    announce("compile fullgraph qk_norm_rope + flash_attn")
    from tinytrain_amd.kernels.flash_attn import flash_attn

    q, k, v, wq, wk, cos, sin = _dev(*_inputs(2, 64, 4, 2, 64))

    def f(q, k, v, wq, wk):
        a, b, c = qk_norm_rope(q, k, v, wq, wk, cos, sin)
        return flash_attn(a, b, c).float().sum()

    ins = [t.clone().requires_grad_() for t in (q, k, v, wq, wk)]
    f(*ins).backward()
    ins2 = [t.clone().requires_grad_() for t in (q, k, v, wq, wk)]
    torch.compile(f, fullgraph=True)(*ins2).backward()
    for a, b in zip(ins, ins2):
        assert torch.equal(a.grad, b.grad)
