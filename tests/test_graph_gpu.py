"""HIP-graph capture of the attention ops.

A forward + backward (and a decode call) captured with torch.cuda.graph replays with
the same results as eager calls on the same inputs, bitwise (the kernels are
deterministic). Each test replays four times with new inputs copied into the captured
buffers, with eager launches and host synchronisations between the replays, and checks
every replay. The library makes no allocation, memset or synchronisation, so a capture
holds only its kernel launches.
"""

import pytest
import torch

from helpers import announce
from tinytrain_amd.kernels.decode import flash_attn_decode
from tinytrain_amd.kernels.flash_attn import _backward, _forward

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _unit_rms(t):
    return t / t.pow(2).mean(-1, keepdim=True).sqrt()


def _attn_inputs(seed, B, Hq, Hkv, T, D):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = _unit_rms(torch.randn(B, Hq, T, D, device=DEV, generator=g)).bfloat16()
    k = _unit_rms(torch.randn(B, Hkv, T, D, device=DEV, generator=g)).bfloat16()
    v = torch.randn(B, Hkv, T, D, device=DEV, generator=g).bfloat16()
    do = (torch.randn(B, Hq, T, D, device=DEV, generator=g) * 1e-2).bfloat16()
    return q, k, v, do


def _capture(fn):
    """Warm up on a side stream (default priority), then capture fn's launches."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


@pytest.mark.parametrize("B,Hq,Hkv,T,D", [(2, 4, 2, 300, 64), (1, 4, 4, 257, 128)])
def test_graph_replay_fwd_bwd(B, Hq, Hkv, T, D):
    announce(f"graph replay fwd+bwd B={B} Hq={Hq} Hkv={Hkv} T={T} D={D}")
    static = _attn_inputs(0, B, Hq, Hkv, T, D)

    def step():
        o, M = _forward(*static[:3])
        return (o, M) + _backward(static[0], static[1], static[2], o, static[3], M)

    graph, out = _capture(step)
    for seed in (1, 2, 3, 4):
        new = _attn_inputs(seed, B, Hq, Hkv, T, D)
        for dst, src in zip(static, new):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        o, M = _forward(*new[:3])
        want = (o, M) + _backward(new[0], new[1], new[2], o, new[3], M)
        torch.cuda.synchronize()
        for name, a, b in zip(("O", "LSE", "dQ", "dK", "dV"), out, want):
            assert torch.equal(a, b), f"replay with seed {seed}: {name} differs from eager"


def test_graph_replay_decode():
    announce("graph replay decode B=4 Hq=8 Hkv=2 Tq=2 L=1024 D=128")
    B, Hq, Hkv, Tq, L, D = 4, 8, 2, 2, 1024, 128

    def inputs(seed):
        g = torch.Generator(device=DEV).manual_seed(seed)
        q = _unit_rms(torch.randn(B, Hq, Tq, D, device=DEV, generator=g)).bfloat16()
        k = _unit_rms(torch.randn(B, Hkv, L, D, device=DEV, generator=g)).bfloat16()
        v = torch.randn(B, Hkv, L, D, device=DEV, generator=g).bfloat16()
        lens = torch.randint(1, L + 1, (B,), device=DEV, generator=g, dtype=torch.int32)
        return q, k, v, lens

    static = inputs(0)
    graph, out = _capture(lambda: flash_attn_decode(*static))
    for seed in (1, 2, 3, 4):
        new = inputs(seed)
        for dst, src in zip(static, new):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        want = flash_attn_decode(*new)
        torch.cuda.synchronize()
        assert torch.equal(out[0], want[0]) and torch.equal(out[1], want[1]), f"seed {seed}"
