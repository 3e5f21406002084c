"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

CPU: the seeded generator reproduces the stored inputs bit for bit and every
workload's input digest; the oracle reproduces the stored outputs.
GPU: the HIP ops on the stored inputs match the stored outputs to the parity
tolerances (O/dQ/dK/dV max-abs 2e-2 bf16, 1e-5 fp32; LSE 1e-3).
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import announce, assert_close_abs
from oracle.eager_attention import TOL, TOL_LSE, max_abs, reference_outputs
from tinytrain_amd.workloads import CONFIGS, digest, make_custom, make_inputs

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = {
    "gqa2_t33_d64_bf16": (1, 2, 1, 33, 64, torch.bfloat16, 21),
    "gqa2_t17_d128_bf16": (1, 4, 2, 17, 128, torch.bfloat16, 22),
    "mha_t40_d64_f32": (1, 2, 2, 40, 64, torch.float32, 23),
}
OUTS = ("o", "lse", "dq", "dk", "dv")


def _load(name):
    with np.load(GOLDEN / "attn_small.npz") as z:
        return {k.split("/", 1)[1]: torch.from_numpy(z[k]) for k in z.files if k.startswith(name + "/")}


@pytest.mark.parametrize("name", sorted(CASES))
def test_generator_reproduces_golden_inputs(name):
    B, Hq, Hkv, T, D, dt, seed = CASES[name]
    g = _load(name)
    q, k, v, do = make_custom(B, Hq, Hkv, T, D, dt, seed=seed)
    for key, t in (("q", q), ("k", k), ("v", v), ("do", do)):
        assert torch.equal(t.float(), g[key]), key


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_golden_outputs(name):
    g = _load(name)
    dt = CASES[name][5]
    q, k, v, do = (g[x].to(dt) for x in ("q", "k", "v", "do"))
    want = reference_outputs(q, k, v, do, dtype=torch.float64)
    for key, w in zip(OUTS, want):
        assert max_abs(w, g[key]) < 1e-6, key  # stored as fp32


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5", "REF112M"])
def test_workload_input_digests(name):
    ref = json.loads((GOLDEN / "input_digests.json").read_text())[name]
    q, k, v, do, ch = make_inputs(CONFIGS[name], seed=0)
    assert ch == ref["outlier_channels"]
    assert digest(q, k, v, do) == ref["sha256"]


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_hip_matches_golden(name):
    from tinytrain_amd.kernels.flash_attn import _backward, _forward

    announce(f"golden {name}")
    g = _load(name)
    dt = CASES[name][5]
    q, k, v, do = (g[x].to(dt).to("cuda") for x in ("q", "k", "v", "do"))
    o, M = _forward(q, k, v)
    dq, dk, dv = _backward(q, k, v, o, do, M)
    torch.cuda.synchronize()
    for key, got in zip(OUTS, (o, M, dq, dk, dv)):
        tol = TOL_LSE if key == "lse" else TOL[dt]
        assert_close_abs(key, got.cpu(), g[key], tol, f"[{name}]")
