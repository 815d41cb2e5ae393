"""The entry points under HIP graph capture (torch.cuda.CUDAGraph).

Nothing in the library synchronizes with the host, allocates, or records a
memset, so a decode step, a prefill forward or a forward and backward (on
index lists that need no device check) can be captured once and replayed.  Each graph is replayed
several times with new inputs written eagerly between replays, and every
replay must equal an eager call on the same inputs bit for bit.  The decode
replays also change the cache lengths and routing: its work split is planned
on the device at each replay, not baked into the graph.  The prefill shapes
are small grids, so the graphs also hold the forward's key-range split and
merge, the backward's dK/dV split and dQ pieces, and their reduce kernels.
"""

import pytest
import torch

from switchattentionkernels_amd import (build_switch_query_indices, switch_gqa_decode_forward,
                                        switch_gqa_prefill_backward, switch_gqa_prefill_forward)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = fn()
    return graph, outs


def test_decode_graph_replays_match_eager():
    b, L, hq, hkv, w = 12, 4096, 32, 8, 512
    g = torch.Generator(device=DEV).manual_seed(41)
    q = torch.randn(b, 1, hq, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(b, L, hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(b, L, hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    lens = torch.randint(1, L + 1, (b,), generator=g, device=DEV, dtype=torch.int32)
    full = torch.rand(b, generator=g, device=DEV) < 0.5

    graph, (o_g, l_g) = _capture(
        lambda: switch_gqa_decode_forward(q, k, v, lens, full, window_size=w))
    for i in range(4):
        q.copy_(torch.randn(q.shape, generator=g, device=DEV).to(torch.bfloat16))
        lens.copy_(torch.randint(1, L + 1, (b,), generator=g, device=DEV, dtype=torch.int32))
        full.copy_(torch.rand(b, generator=g, device=DEV) < 0.5)
        graph.replay()
        o_e, l_e = switch_gqa_decode_forward(q, k, v, lens, full, window_size=w)
        torch.cuda.synchronize()
        assert torch.equal(o_g, o_e) and torch.equal(l_g, l_e), f"decode replay {i}"


def test_prefill_forward_graph_replays_match_eager():
    s, hq, hkv, w = 2048, 32, 8, 256
    g = torch.Generator(device=DEV).manual_seed(42)
    q = torch.randn(1, s, hq, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(1, s, hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(1, s, hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    full, local = build_switch_query_indices(torch.rand(1, s, generator=g, device=DEV) < 0.3)

    graph, (o_g, l_g) = _capture(
        lambda: switch_gqa_prefill_forward(q, k, v, full, local, window_size=w))
    for i in range(4):
        q.copy_(torch.randn(q.shape, generator=g, device=DEV).to(torch.bfloat16))
        v.copy_(torch.randn(v.shape, generator=g, device=DEV).to(torch.bfloat16))
        graph.replay()
        o_e, l_e = switch_gqa_prefill_forward(q, k, v, full, local, window_size=w)
        torch.cuda.synchronize()
        assert torch.equal(o_g, o_e) and torch.equal(l_g, l_e), f"prefill replay {i}"


def test_prefill_forward_backward_graph_replays_match_eager():
    s, hq, hkv, w = 1536, 16, 4, 300
    g = torch.Generator(device=DEV).manual_seed(43)
    q = torch.randn(1, s, hq, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(1, s, hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(1, s, hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    do = torch.randn(1, s, hq, 128, generator=g, device=DEV).to(torch.bfloat16)
    full, local = build_switch_query_indices(torch.rand(1, s, generator=g, device=DEV) < 0.4)

    def step():
        o, lse = switch_gqa_prefill_forward(q, k, v, full, local, window_size=w)
        return (o, lse) + switch_gqa_prefill_backward(q, k, v, o, lse, do, full, local,
                                                      window_size=w)

    graph, outs_g = _capture(step)
    for i in range(4):
        for t in (q, k, do):
            t.copy_(torch.randn(t.shape, generator=g, device=DEV).to(torch.bfloat16))
        graph.replay()
        outs_e = step()
        torch.cuda.synchronize()
        for name, a, b in zip(("o", "lse", "dq", "dk", "dv"), outs_g, outs_e):
            assert torch.equal(a, b), f"forward+backward replay {i}: {name}"

