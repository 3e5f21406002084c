"""Writes the attention golden fixtures in this directory.

    python tests/golden/make_golden.py

* ``attn_small.npz``: three tiny causal cases (inputs as drawn by the seeded
  generator, outputs O / LSE / dQ / dK / dV of the fp64 oracle).  Inputs of the bf16
  cases are stored as their bf16 values widened to float32, so they round-trip exactly.
* ``input_digests.json``: SHA-256 of each workload's seeded inputs (q, k, v, dO), so a
  change of the generator or of torch's RNG is caught before it silently moves every
  comparison.

The reference (XinqiWan412/tinytrain) holds no attention vectors of its own; these are
produced by this repository's oracle, whose correctness is pinned separately by
tests/test_oracle.py (closed forms, independent implementations, finite differences).
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from oracle.eager_attention import reference_outputs  # noqa: E402
from tinytrain_amd.workloads import CONFIGS, digest, make_custom, make_inputs  # noqa: E402

# (name, B, Hq, Hkv, T, D, dtype, seed)
CASES = [
    ("gqa2_t33_d64_bf16", 1, 2, 1, 33, 64, torch.bfloat16, 21),
    ("gqa2_t17_d128_bf16", 1, 4, 2, 17, 128, torch.bfloat16, 22),
    ("mha_t40_d64_f32", 1, 2, 2, 40, 64, torch.float32, 23),
]


def small_cases():
    out = {}
    for name, B, Hq, Hkv, T, D, dt, seed in CASES:
        q, k, v, do = make_custom(B, Hq, Hkv, T, D, dt, seed=seed)
        o, lse, dq, dk, dv = reference_outputs(q, k, v, do, dtype=torch.float64)
        for key, t in (("q", q), ("k", k), ("v", v), ("do", do)):
            out[f"{name}/{key}"] = t.float().numpy()
        for key, t in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
            out[f"{name}/{key}"] = t.float().numpy()  # fp64 oracle, stored as fp32
    return out


def input_digests():
    res = {}
    for name, cfg in CONFIGS.items():
        q, k, v, do, ch = make_inputs(cfg, seed=0)
        res[name] = {"sha256": digest(q, k, v, do), "outlier_channels": ch}
    return res


if __name__ == "__main__":
    np.savez_compressed(HERE / "attn_small.npz", **small_cases())
    (HERE / "input_digests.json").write_text(json.dumps(input_digests(), indent=1) + "\n")
    print("wrote", HERE / "attn_small.npz", HERE / "input_digests.json")
