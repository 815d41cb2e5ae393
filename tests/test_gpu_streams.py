"""The entry points on two streams at once.

The library keeps no state between calls: each call gets its own workspace
and launches on the stream it is given.  Two problems run concurrently on
two torch streams (default priority) must give exactly what they give one
after the other on the default stream.
"""

import pytest
import torch

from switchattentionkernels_amd import (build_switch_query_indices, switch_gqa_decode_forward,
                                        switch_gqa_prefill_backward, switch_gqa_prefill_forward)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _problem(seed, s=3000, hq=32, hkv=8):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(1, s, hq, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(1, s, hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(1, s, hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    do = torch.randn(1, s, hq, 128, generator=g, device=DEV).to(torch.bfloat16)
    mask = torch.rand(1, s, generator=g, device=DEV) < 0.3
    kc = torch.randn(16, 2048, hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(16, 2048, hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    qd = torch.randn(16, hq, 128, generator=g, device=DEV).to(torch.bfloat16)
    lens = torch.randint(0, 2049, (16,), generator=g, device=DEV, dtype=torch.int32)
    full = torch.rand(16, generator=g, device=DEV) < 0.5
    return q, k, v, do, mask, qd, kc, vc, lens, full


def _run(pb, w=512):
    q, k, v, do, mask, qd, kc, vc, lens, full = pb
    f, l = build_switch_query_indices(mask)
    o, lse = switch_gqa_prefill_forward(q, k, v, f, l, window_size=w)
    dq, dk, dv = switch_gqa_prefill_backward(q, k, v, o, lse, do, f, l, window_size=w)
    od, ld = switch_gqa_decode_forward(qd, kc, vc, lens, full, window_size=w)
    return o, lse, dq, dk, dv, od, ld


def test_two_streams_match_sequential():
    a, b = _problem(101), _problem(202)
    ref_a, ref_b = _run(a), _run(b)
    torch.cuda.synchronize()
    main = torch.cuda.current_stream()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(main)
    s2.wait_stream(main)
    for _ in range(3):
        with torch.cuda.stream(s1):
            got_a = _run(a)
        with torch.cuda.stream(s2):
            got_b = _run(b)
        torch.cuda.synchronize()
        names = ("o", "lse", "dq", "dk", "dv", "decode o", "decode lse")
        for name, x, y in zip([f"a {n}" for n in names] + [f"b {n}" for n in names],
                              got_a + got_b, ref_a + ref_b):
            assert torch.equal(x, y) or (torch.isnan(x).equal(torch.isnan(y)) and
                                         torch.equal(torch.nan_to_num(x), torch.nan_to_num(y))), name
