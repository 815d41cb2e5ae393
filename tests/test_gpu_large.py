"""Tensors past 2^31 bytes and elements: 64-bit addressing in the forward and
backward kernels.

B1 S131072 Hq128/Hkv16 (G = 8) d128, W 2048, p_full 0.25: Q, O and dO hold
2^31 elements (4 GiB each), so rows in the second half sit past byte offset
2^31 and the last rows at element offsets near 2^31.  Inputs are drawn on the
GPU from a seeded generator.  Sampled rows, most of them in the last quarter,
are checked against the oracle, which runs on just those rows: a sub-problem
of the sampled query rows with their original key bounds passed as position
metadata (full rows [0, p], local rows [p - W + 1, p], F:145-155) over the
full K and V.  Bars as elsewhere: O max-abs <= 2e-2, mean-abs <= 2e-3, LSE
relative <= 1e-3; dq, and dK / dV of the last 64 keys, relative L2 <= 1e-2,
relative max <= 3e-2.
"""

import numpy as np
import pytest
import torch

import oracle
from switchattentionkernels_amd import (build_switch_query_indices, switch_gqa_prefill_backward,
                                        switch_gqa_prefill_forward)

pytestmark = pytest.mark.gpu
DEV = "cuda"
S, HQ, HKV, W = 131072, 128, 16, 2048


def _sub_problem(mask_np, pos):
    """Routing lists and key bounds of the sampled rows as a stand-alone problem."""
    f = mask_np[pos]
    md = {"full_starts": np.zeros(pos.size, dtype=np.int64),
          "local_starts": np.maximum(pos - W + 1, 0),
          "causal_ends": pos + 1}
    return np.nonzero(f)[0], np.nonzero(~f)[0], md


def test_tensors_past_2gib_sampled_rows():
    g = torch.Generator(device=DEV).manual_seed(21)
    q = torch.randn(1, S, HQ, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(1, S, HKV, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(1, S, HKV, 128, generator=g, device=DEV).to(torch.bfloat16)
    mask = torch.rand(1, S, generator=g, device=DEV) < 0.25
    assert q.numel() * q.element_size() >= 2 ** 32
    print(f"[large] S{S} Hq{HQ}/Hkv{HKV} W{W}: forward", flush=True)
    full, local = build_switch_query_indices(mask)
    o, lse = switch_gqa_prefill_forward(q, k, v, full, local, window_size=W)
    torch.cuda.synchronize()

    rng = np.random.default_rng(21)
    pos = np.unique(np.concatenate([rng.integers(3 * S // 4, S, 20), [0, S // 2, S - 1]]))
    mask_np = mask[0].cpu().numpy()
    fi, li, md = _sub_problem(mask_np, pos)
    kc, vc = k.cpu(), v.cpu()
    qs = q[0, torch.as_tensor(pos, device=DEV)].unsqueeze(0).cpu()
    o_ref, lse_ref = oracle.routed_attention(qs, kc, vc, fi, li, window_size=W, metadata=md)
    o_got = o[0, torch.as_tensor(pos, device=DEV)].float().cpu()
    l_got = lse[0, torch.as_tensor(pos, device=DEV)].cpu()
    err = (o_got - o_ref[0]).abs()
    lerr = ((l_got - lse_ref[0]).abs() / lse_ref[0].abs().clamp(min=1.0)).max().item()
    print(f"[large] forward: O max {err.max().item():.3e} mean {err.mean().item():.3e} "
          f"LSE rel {lerr:.3e}", flush=True)
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3 and lerr <= 1e-3

    print("[large] backward", flush=True)
    do = torch.randn(1, S, HQ, 128, generator=g, device=DEV).to(torch.bfloat16)
    dq, dk, dv = switch_gqa_prefill_backward(q, k, v, o, lse, do, full, local, window_size=W)
    torch.cuda.synchronize()
    assert torch.isfinite(dk).all() and torch.isfinite(dv).all()
    pb = pos[-8:]
    fi, li, md = _sub_problem(mask_np, pb)
    sel = torch.as_tensor(pb, device=DEV)
    rq, _, _ = oracle.routed_attention_backward(q[0, sel].unsqueeze(0).cpu(), kc, vc,
                                                do[0, sel].unsqueeze(0).cpu(), fi, li,
                                                window_size=W, metadata=md)
    got = dq[0, sel].float().cpu()
    e = got - rq[0]
    l2 = float(e.norm() / rq[0].norm())
    mx = float(e.abs().max() / rq[0].abs().max())
    print(f"[large] dq sampled rows: rel_l2 {l2:.2e} rel_max {mx:.2e}", flush=True)
    assert l2 <= 1e-2 and mx <= 3e-2

    # dK / dV of the last `late` keys: only rows at the last `late` positions
    # see them (causal, and W > late), so those rows as a stand-alone problem
    # over the full K / V give these keys' gradients exactly.  The dK/dV
    # kernel gathers those Q / dO rows from byte offsets near 2^32.
    late = 64
    pl = np.arange(S - late, S)
    assert mask_np[pl].any() and (~mask_np[pl]).any()
    fi, li, md = _sub_problem(mask_np, pl)
    sel = torch.as_tensor(pl, device=DEV)
    _, rk, rv = oracle.routed_attention_backward(q[0, sel].unsqueeze(0).cpu(), kc, vc,
                                                 do[0, sel].unsqueeze(0).cpu(), fi, li,
                                                 window_size=W, metadata=md, chunk=8)
    for name, got, ref in (("dk", dk, rk), ("dv", dv, rv)):
        g_ = got[0, S - late:].float().cpu()
        r_ = ref[0, S - late:]
        e = g_ - r_
        l2 = float(e.norm() / r_.norm())
        mx = float(e.abs().max() / r_.abs().max())
        print(f"[large] {name} of the last {late} keys: rel_l2 {l2:.2e} rel_max {mx:.2e}",
              flush=True)
        assert l2 <= 1e-2 and mx <= 3e-2


def test_decode_caches_past_2gib():
    """Decode over [16, 131072, 8, 128] caches (4 GiB each, 2^31 elements):
    the last sequences' keys sit past byte offset 3 GiB.  The oracle runs per
    sequence on the routed slice of its cache ([lo, n) as a whole cache of
    n - lo keys, routed full), which is the same problem."""
    from switchattentionkernels_amd import switch_gqa_decode_forward
    b, L, hq, hkv, w = 16, 131072, 32, 8, 4096
    g = torch.Generator(device=DEV).manual_seed(22)
    q = torch.randn(b, hq, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(b, L, hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(b, L, hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    assert k.numel() * k.element_size() >= 2 ** 32
    lens = [1, 5000, 9000, 70000, 30, L, 100, 64, 4097, 4096, 20000, 77777, 3, L - 1, 100000, L]
    full = [True, False, False, True, False, True, True, False,
            False, True, False, True, False, False, True, True]
    print(f"[large] decode B{b} L{L} Hq{hq}/Hkv{hkv} W{w}", flush=True)
    o, lse = switch_gqa_decode_forward(q, k, v, torch.tensor(lens, dtype=torch.int32, device=DEV),
                                       torch.tensor(full, device=DEV), window_size=w)
    torch.cuda.synchronize()
    o, lse = o.float().cpu(), lse.cpu()
    worst = 0.0
    for i in range(b):
        n = lens[i]
        lo = 0 if full[i] else max(n - w, 0)
        o_r, lse_r = oracle.decode_attention(q[i:i + 1].cpu(), k[i:i + 1, lo:n].cpu(),
                                             v[i:i + 1, lo:n].cpu(), [n - lo], [True],
                                             window_size=w)
        err = (o[i] - o_r[0]).abs()
        lerr = ((lse[i] - lse_r[0]).abs() / lse_r[0].abs().clamp(min=1.0)).max().item()
        assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3 and lerr <= 1e-3, (
            f"sequence {i}: O max {err.max().item():.3e} mean {err.mean().item():.3e} "
            f"LSE rel {lerr:.3e}")
        worst = max(worst, err.max().item())
    print(f"[large] decode: worst O max-abs {worst:.3e}", flush=True)
