"""Whole-model logits at the reference's 112M pretrain shape, hip vs sdpa vs fp32.

The reference's model test compares the attention switch's logits under bf16 autocast
(tests/test_flash_attn.py:128-140).  At the 112M shape (12 layers, H=8, H_kv=2, D=128,
T=512, model.py defaults) the bf16 autocast path is itself noisy: sdpa in bf16 differs
from the same model in fp32 by a few hundredths in the logits.  So the bound here is
relative to that noise: with the HIP attention, the model's bf16 logits must be as
close to the fp32 reference (sdpa, no autocast) as the sdpa path's own bf16 logits
are, within a small factor, eager and under torch.compile.

A broken kernel (a wrong mask, scale or GQA head map) moves the logits by far more than
the bf16 noise, so the bound still catches it.
"""

import pytest
import torch

from helpers import announce
from tinytrain_amd.model import ModelConfig, ModelForCausalLM

pytestmark = pytest.mark.gpu

DEV = "cuda"
# hip's deviation from the fp32 logits, as a multiple of sdpa-bf16's own deviation.  The
# mean is the tight bound: it measured 0.996-1.002 on every box.  The maximum is set by a
# handful of logits.  Eager, every kernel is deterministic and the ratio of the maxima is
# bounded as tightly as the mean's spread allows.  Compiled, the generated kernels around
# the attention ops round differently from box to box: the ratio of the maxima read
# 0.97-1.02 on one box and 1.16 on another for the same code (the per-box values are
# kept in profiles/model_112m_logits.txt), so that bound leaves room for the spread.  A
# wrong mask, scale or head map moves both far beyond these bounds.
MAX_RATIO_EAGER = 1.15
MAX_RATIO_COMPILED = 1.5
MEAN_RATIO = 1.05


@pytest.fixture(scope="module")
def model_112m():
    torch.manual_seed(0)
    c = ModelConfig()
    assert (c.num_attention_heads, c.num_key_value_heads, c.head_dim, c.max_seq_len) == (8, 2, 128, 512)
    model = ModelForCausalLM(c).to(DEV).eval()
    g = torch.Generator(device="cpu").manual_seed(1)
    x = torch.randint(0, c.vocab_size, (2, c.max_seq_len), generator=g).to(DEV)
    model.set_attn_impl("sdpa")
    with torch.no_grad():
        ref = model(x)[0].float()  # fp32 throughout, eager sdpa
    yield model, x, ref
    torch._dynamo.reset()


def _logits(model, x, impl, fused=False, compiled=False):
    model.set_attn_impl(impl, fused_prologue=fused)
    m = model
    if compiled:
        torch._dynamo.reset()
        m = torch.compile(model)
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        out = m(x)[0].float()
    torch.cuda.synchronize()
    return out


def _check(name, got, sdpa, ref, max_ratio):
    e_hip, e_sdpa = (got - ref).abs(), (sdpa - ref).abs()
    msg = (f"{name}: |hip - fp32| max {e_hip.max().item():.5f} mean {e_hip.mean().item():.6f}; "
           f"|sdpa_bf16 - fp32| max {e_sdpa.max().item():.5f} mean {e_sdpa.mean().item():.6f}; "
           f"ratios max {(e_hip.max() / e_sdpa.max()).item():.4f} "
           f"mean {(e_hip.mean() / e_sdpa.mean()).item():.4f}")
    print(msg, flush=True)
    assert torch.isfinite(got).all(), msg
    assert e_hip.max() <= max_ratio * e_sdpa.max(), msg
    assert e_hip.mean() <= MEAN_RATIO * e_sdpa.mean(), msg


def test_112m_logits_eager(model_112m):
    announce("112M logits eager: hip, hip + fused prologue vs sdpa bf16 vs fp32")
    model, x, ref = model_112m
    sdpa = _logits(model, x, "sdpa")
    _check("hip eager", _logits(model, x, "hip"), sdpa, ref, MAX_RATIO_EAGER)
    _check("hip + fused prologue eager", _logits(model, x, "hip", fused=True), sdpa, ref,
           MAX_RATIO_EAGER)


def test_112m_logits_compiled(model_112m):
    announce("112M logits torch.compile: hip vs sdpa bf16 vs fp32")
    model, x, ref = model_112m
    sdpa = _logits(model, x, "sdpa", compiled=True)
    _check("hip compiled", _logits(model, x, "hip", compiled=True), sdpa, ref,
           MAX_RATIO_COMPILED)
