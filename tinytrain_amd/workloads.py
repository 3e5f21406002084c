"""The five attention workloads and their seeded synthetic inputs.

Used by bench.py (the timed inputs), by the tests and by the CPU oracle's checks, so
every consumer sees the same bits.  The same bits are produced on every host: everything is drawn on the CPU from
``torch.Generator("cpu").manual_seed(seed)`` in the order q, k, v, dO (the seed 0 and
the randn-per-tensor pattern follow tests/test_flash_attn.py:16-21), then normalised,
then cast, and only then moved to a device.

"Unit-RMS per head along D" is x * rsqrt(mean(x^2, -1) + 1e-6), the RMSNorm of
model.py:30-35 with unit weight (the q/k-norm applied before attention in
model.py:87).
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass
from typing import Dict

import torch


@dataclass(frozen=True)
class AttnConfig:
    name: str
    B: int
    Hq: int
    Hkv: int
    T: int
    D: int
    dtype: torch.dtype
    qkv_unit_rms: str       # which of q, k, v are RMS-normalised ("qkv" or "qk")
    do_scale: float         # dO ~ N(0,1) * do_scale
    outlier_frac: float = 0.0   # fraction of D channels of q and k scaled by outlier_gain
    outlier_gain: float = 8.0

    @property
    def group(self) -> int:
        return self.Hq // self.Hkv

    def fwd_flop(self) -> float:
        """Causal forward FLOPs, FA convention: 4*B*Hq*T^2*D / 2 (two matmuls, half masked)."""
        return 2.0 * self.B * self.Hq * self.T * self.T * self.D

    def bwd_flop(self) -> float:
        """Backward = 2.5 x forward (five matmuls: S recompute, dP, dV, dQ, dK)."""
        return 2.5 * self.fwd_flop()


# The BASELINE.json workload table (configs[0..4]).
CONFIGS: Dict[str, AttnConfig] = {
    "C1": AttnConfig("C1", 2, 4, 4, 256, 64, torch.float32, "qkv", 1.0),
    "C2": AttnConfig("C2", 16, 12, 12, 1024, 64, torch.bfloat16, "qk", 1e-2),
    "C3": AttnConfig("C3", 32, 12, 4, 1024, 64, torch.bfloat16, "qk", 1e-2),
    "C4": AttnConfig("C4", 4, 16, 8, 4096, 128, torch.bfloat16, "qk", 1e-2, outlier_frac=0.01),
    "C5": AttnConfig("C5", 1, 16, 8, 16384, 128, torch.bfloat16, "qk", 1e-2),
    # The reference model's own attention shape (model.py:11-18: 8 query heads, 2 KV heads,
    # head_dim 128, max_seq_len 512) at the batch its attn_impl comparison is quoted on
    # (docs/results.md:184, B=32); inputs drawn like C2.
    "REF112M": AttnConfig("REF112M", 32, 8, 2, 512, 128, torch.bfloat16, "qk", 1e-2),
}

def unit_rms(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps) along the last dim, in fp32 (model.py:33-34)."""
    x = x.float()
    return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)


def make_inputs(cfg: AttnConfig, seed: int = 0, batch: int | None = None):
    """(q, k, v, do) on the CPU in ``cfg.dtype`` plus the outlier channel list.

    ``batch`` < cfg.B draws only the first ``batch`` sequences (same bits as the
    leading slice of the full draw, because each tensor is drawn whole and sliced).
    """
    g = torch.Generator("cpu").manual_seed(seed)
    B, Hq, Hkv, T, D = cfg.B, cfg.Hq, cfg.Hkv, cfg.T, cfg.D
    q = torch.randn(B, Hq, T, D, generator=g)
    k = torch.randn(B, Hkv, T, D, generator=g)
    v = torch.randn(B, Hkv, T, D, generator=g)
    do = torch.randn(B, Hq, T, D, generator=g) * cfg.do_scale
    q, k = unit_rms(q), unit_rms(k)
    if "v" in cfg.qkv_unit_rms:
        v = unit_rms(v)
    channels: list[int] = []
    if cfg.outlier_frac > 0:
        n = max(1, round(cfg.outlier_frac * D))
        channels = torch.randperm(D, generator=g)[:n].tolist()
        q[..., channels] *= cfg.outlier_gain
        k[..., channels] *= cfg.outlier_gain
    if batch is not None:
        q, k, v, do = q[:batch], k[:batch], v[:batch], do[:batch]
    out = tuple(t.to(cfg.dtype).contiguous() for t in (q, k, v, do))
    return out + (channels,)


def make_custom(B: int, Hq: int, Hkv: int, T: int, D: int, dtype=torch.bfloat16,
                seed: int = 0, do_scale: float = 1.0):
    """Plain N(0,1) inputs of any shape (the reference test's generator,
    tests/test_flash_attn.py:16-21, but drawn on the CPU)."""
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, Hq, T, D, generator=g)
    k = torch.randn(B, Hkv, T, D, generator=g)
    v = torch.randn(B, Hkv, T, D, generator=g)
    do = torch.randn(B, Hq, T, D, generator=g) * do_scale
    return tuple(t.to(dtype).contiguous() for t in (q, k, v, do))


def digest(*tensors: torch.Tensor) -> str:
    """SHA-256 over the raw bytes of the tensors (detects RNG or generator drift)."""
    h = hashlib.sha256()
    for t in tensors:
        t = t.contiguous()
        if t.dtype == torch.bfloat16:
            t = t.view(torch.int16)
        h.update(t.numpy().tobytes())
    return h.hexdigest()
