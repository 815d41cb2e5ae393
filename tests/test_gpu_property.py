"""Property-based sweeps over small shapes (hypothesis): the HIP forward, the
HIP backward, packed sequences (forward and backward), the compaction (from
a mask and from router logits), the routed decode, split-then-merged key
ranges, the forward on arbitrary caller key bounds, the backward on
monotone caller key bounds, and small grids that take the forward's
key-range split and the backward's dQ pieces, against the CPU oracle.

The examples are derandomized: every run draws the same fixed set of shapes
(batch, lengths, head counts, group size, window, routing density, key
length), so a failure names a reproducible case.  Bars as in the fixed-shape
parity tests: O max-abs <= 2e-2, mean-abs <= 2e-3, LSE relative <= 1e-3,
compaction bit-exact; gradients relative L2 <= 1e-2 and relative max <= 3e-2,
each measured against max(|g_ref|, 1e-2) so that a gradient that is zero in
exact arithmetic (a row that sees a single key) is held to an absolute bar.
The gradient reference takes Delta = dO . O from the kernel's own bf16
forward output, as the kernel does (the FlashAttention-2 convention): rows
with one or two legal keys can otherwise sit just above 1e-2 by the known
Delta shift (tests/test_gpu_backward.py bounds that shift against the exact
gradient); the fixed-shape backward tests compare with the exact gradient.
"""

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import oracle
from oracle import routing as R
from switchattentionkernels_amd import (build_switch_attention_metadata,
                                        build_switch_query_indices,
                                        build_switch_query_indices_from_logits,
                                        switch_gqa_decode_forward,
                                        switch_gqa_prefill_backward, switch_gqa_prefill_forward,
                                        switch_gqa_prefill_varlen_forward, workloads)

from test_gpu_parity import _assert_close, _split_run

pytestmark = pytest.mark.gpu
DEV = "cuda"

SETTINGS = dict(deadline=None, derandomize=True, database=None,
                suppress_health_check=list(HealthCheck))

shapes = st.fixed_dictionaries({
    "b": st.integers(1, 2),
    "s": st.integers(1, 320),
    "hkv": st.integers(1, 3),
    "g": st.sampled_from([1, 2, 4, 5, 8]),
    "w": st.integers(1, 400),
    "p": st.sampled_from([0.0, 0.1, 0.5, 0.9, 1.0]),
    "dkv": st.integers(-120, 120),
    "seed": st.integers(0, 2 ** 16),
})


def _case(c):
    skv = max(1, c["s"] + c["dkv"])
    gen = torch.Generator().manual_seed(c["seed"])
    hq = c["g"] * c["hkv"]
    q, k, v = workloads.make_qkv(gen, c["b"], c["s"], skv, hq, c["hkv"], 128)
    mask = torch.rand((c["b"], c["s"]), generator=gen) < c["p"]
    tag = (f"b{c['b']} s{c['s']} skv{skv} {hq}/{c['hkv']} w{c['w']} p{c['p']} "
           f"seed{c['seed']}")
    print(f"[property] {tag}", flush=True)
    return q, k, v, mask, gen, tag


@settings(max_examples=80, **SETTINGS)
@given(c=shapes)
def test_forward_property(c):
    q, k, v, mask, _, tag = _case(c)
    full, local = build_switch_query_indices(mask.to(DEV))
    o, lse = switch_gqa_prefill_forward(q.to(DEV), k.to(DEV), v.to(DEV), full, local,
                                        window_size=c["w"])
    torch.cuda.synchronize()
    f_np, l_np = R.compact(mask.numpy())
    o_ref, lse_ref = oracle.routed_attention(q, k, v, f_np, l_np, window_size=c["w"])
    _assert_close(o, lse, o_ref, lse_ref, tag=tag)


def _grad_close(got, ref, tag):
    got, ref = got.float().cpu(), ref.float()
    assert torch.isfinite(got).all(), f"{tag}: non-finite gradient"
    err = got - ref
    floor = 1e-2
    l2 = float(err.norm() / max(float(ref.norm()), floor * ref.numel() ** 0.5))
    mx = float(err.abs().max() / max(float(ref.abs().max()), floor))
    assert l2 <= 1e-2 and mx <= 3e-2, f"{tag}: rel_l2 {l2:.3e} rel_max {mx:.3e}"


@settings(max_examples=40, **SETTINGS)
@given(c=shapes)
def test_backward_property(c):
    q, k, v, mask, gen, tag = _case(c)
    do = torch.randn(q.shape, generator=gen).to(torch.bfloat16)
    full, local = build_switch_query_indices(mask.to(DEV))
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = switch_gqa_prefill_forward(qd, kd, vd, full, local, window_size=c["w"])
    grads = switch_gqa_prefill_backward(qd, kd, vd, o, lse, do.to(DEV), full, local,
                                        window_size=c["w"])
    torch.cuda.synchronize()
    f_np, l_np = R.compact(mask.numpy())
    refs = oracle.routed_attention_backward(q, k, v, do, f_np, l_np, window_size=c["w"],
                                            out=o.cpu())
    for name, g, r in zip(("dq", "dk", "dv"), grads, refs):
        _grad_close(g, r, f"{tag} {name}")


@settings(max_examples=60, **SETTINGS)
@given(b=st.integers(1, 4), s=st.integers(1, 40000), p=st.floats(0.0, 1.0), seed=st.integers(0, 2 ** 16))
def test_compaction_property(b, s, p, seed):
    mask = torch.rand((b, s), generator=torch.Generator().manual_seed(seed)) < p
    full, local = build_switch_query_indices(mask.to(DEV))
    flat = mask.reshape(-1)
    assert torch.equal(full.cpu(), torch.nonzero(flat).flatten().to(torch.int32))
    assert torch.equal(local.cpu(), torch.nonzero(~flat).flatten().to(torch.int32))


@settings(max_examples=40, **SETTINGS)
@given(b=st.integers(1, 3), s=st.integers(1, 30000),
       dtype=st.sampled_from([torch.float32, torch.bfloat16, torch.float16]),
       thr=st.floats(-2.0, 2.0), special=st.floats(0.0, 0.05), seed=st.integers(0, 2 ** 16))
def test_logits_compaction_property(b, s, dtype, thr, special, seed):
    """Routing from logits in one pass equals thresholding then compacting,
    bit for bit, with NaN and +-inf sprinkled in."""
    gen = torch.Generator().manual_seed(seed)
    lg = torch.randn((b, s), generator=gen) * 1.5
    u = torch.rand((b, s), generator=gen)
    lg[u < special / 3] = float("nan")
    lg[(u >= special / 3) & (u < 2 * special / 3)] = float("inf")
    lg[(u >= 2 * special / 3) & (u < special)] = float("-inf")
    d = lg.to(dtype).to(DEV)
    f, l = build_switch_query_indices_from_logits(d, thr)
    f_ref, l_ref = build_switch_query_indices(d > thr)
    assert torch.equal(f, f_ref) and torch.equal(l, l_ref), (b, s, dtype, thr, seed)


@settings(max_examples=60, **SETTINGS)
@given(c=st.fixed_dictionaries({
    "b": st.integers(1, 40),
    "cache": st.integers(1, 3000),
    "hkv": st.integers(1, 3),
    "g": st.sampled_from([1, 2, 3, 4, 5, 8]),
    "w": st.integers(1, 2000),
    "p": st.sampled_from([0.0, 0.3, 1.0]),
    "empty": st.sampled_from([0.0, 0.2]),
    "seed": st.integers(0, 2 ** 16),
}))
def test_decode_property(c):
    """Routed decode over random cache lengths (some empty), group sizes,
    windows and routing, against the oracle."""
    gen = torch.Generator().manual_seed(c["seed"])
    b, cache, hkv = c["b"], c["cache"], c["hkv"]
    hq = c["g"] * hkv
    q = torch.randn(b, hq, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(b, cache, hkv, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(b, cache, hkv, 128, generator=gen).to(torch.bfloat16)
    lens = torch.randint(0, cache + 1, (b,), generator=gen)
    lens[torch.rand(b, generator=gen) < c["empty"]] = 0
    full = torch.rand(b, generator=gen) < c["p"]
    tag = f"decode b{b} cache{cache} {hq}/{hkv} w{c['w']} p{c['p']} seed{c['seed']}"
    print(f"[property] {tag}", flush=True)
    o, lse = switch_gqa_decode_forward(q.to(DEV), k.to(DEV), v.to(DEV),
                                       lens.to(torch.int32).to(DEV), full.to(DEV),
                                       window_size=c["w"])
    o_r, lse_r = oracle.decode_attention(q, k, v, lens.tolist(), full.tolist(),
                                         window_size=c["w"])
    _assert_close(o.unsqueeze(1), lse.unsqueeze(1), o_r.unsqueeze(1), lse_r.unsqueeze(1), tag=tag)


@settings(max_examples=40, **SETTINGS)
@given(c=st.fixed_dictionaries({
    "s": st.integers(2, 600),
    "hkv": st.integers(1, 2),
    "g": st.sampled_from([1, 4, 5]),
    "w": st.integers(1, 700),
    "p": st.sampled_from([0.0, 0.3, 1.0]),
    "cuts": st.lists(st.floats(0.02, 0.98), min_size=1, max_size=3),
    "seed": st.integers(0, 2 ** 16),
}))
def test_split_merge_property(c):
    """Keys cut into 2-4 chunks at random points: each chunk attended with
    shard metadata, the partials merged by their log2 LSE, equals the
    oracle on the whole key range."""
    s, hkv = c["s"], c["hkv"]
    hq = c["g"] * hkv
    gen = torch.Generator().manual_seed(c["seed"])
    q, k, v = workloads.make_qkv(gen, 1, s, s, hq, hkv, 128)
    mask = torch.rand((1, s), generator=gen) < c["p"]
    cuts = sorted({min(max(int(f * s), 1), s - 1) for f in c["cuts"]})
    bounds = [0] + cuts + [s]
    chunks = tuple(zip(bounds[:-1], bounds[1:]))
    tag = f"split s{s} {hq}/{hkv} w{c['w']} p{c['p']} chunks{chunks} seed{c['seed']}"
    print(f"[property] {tag}", flush=True)
    full, local = build_switch_query_indices(mask.to(DEV))
    pos = torch.arange(s, dtype=torch.int32, device=DEV)
    o, lse = _split_run(q.to(DEV), k.to(DEV), v.to(DEV), full, local, pos, chunks, c["w"])
    f_ref, l_ref = R.compact(mask.reshape(-1).numpy())
    o_r, lse_r = oracle.routed_attention(q, k, v, f_ref, l_ref, window_size=c["w"])
    _assert_close(o, lse, o_r, lse_r, tag=tag)


@settings(max_examples=40, **SETTINGS)
@given(c=st.fixed_dictionaries({
    "lens": st.lists(st.integers(1, 250), min_size=1, max_size=5),
    "hkv": st.integers(1, 2),
    "g": st.sampled_from([1, 4, 5, 8]),
    "w": st.integers(1, 300),
    "p": st.sampled_from([0.0, 0.3, 1.0]),
    "seed": st.integers(0, 2 ** 16),
}))
def test_varlen_property(c):
    """Packed sequences of random lengths (cu_seqlens): forward through
    switch_gqa_prefill_varlen_forward and backward with the same metadata,
    against the oracle on the restated per-segment bounds."""
    cu = [0]
    for n in c["lens"]:
        cu.append(cu[-1] + n)
    t, hkv = cu[-1], c["hkv"]
    hq = c["g"] * hkv
    gen = torch.Generator().manual_seed(c["seed"])
    q, k, v = workloads.make_qkv(gen, 1, t, t, hq, hkv, 128)
    mask = torch.rand((1, t), generator=gen) < c["p"]
    do = torch.randn(q.shape, generator=gen).to(torch.bfloat16)
    tag = f"varlen cu{cu} {hq}/{hkv} w{c['w']} p{c['p']} seed{c['seed']}"
    print(f"[property] {tag}", flush=True)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    full, local = build_switch_query_indices(mask.to(DEV))
    o, lse = switch_gqa_prefill_varlen_forward(qd, kd, vd, full, local, cu, window_size=c["w"])
    md = build_switch_attention_metadata(t, t, device=DEV, window_size=c["w"], cu_seqlens=cu)
    grads = switch_gqa_prefill_backward(qd, kd, vd, o, lse, do.to(DEV), full, local,
                                        metadata=md, window_size=c["w"])
    torch.cuda.synchronize()
    ref_md = R.varlen_metadata(cu, cu, c["w"])
    f_np, l_np = R.compact(mask.numpy())
    o_ref, lse_ref = oracle.routed_attention(q, k, v, f_np, l_np, metadata=ref_md)
    _assert_close(o, lse, o_ref, lse_ref, tag=tag)
    refs = oracle.routed_attention_backward(q, k, v, do, f_np, l_np, metadata=ref_md,
                                            out=o.cpu())
    for name, g, r in zip(("dq", "dk", "dv"), grads, refs):
        _grad_close(g, r, f"{tag} {name}")



def _metadata(fs, ls, ce, s, skv):
    """Caller-made position metadata for one sequence of s queries over skv keys."""
    from switchattentionkernels_amd.metadata import SwitchAttentionMetadata
    i32 = lambda a: torch.as_tensor(np.asarray(a, dtype=np.int32), device=DEV)
    return SwitchAttentionMetadata(i32(np.arange(s)), i32(np.arange(skv)), i32(np.zeros(s)),
                                   i32(np.zeros(skv)), i32(fs), i32(ls), i32(ce))


bounds_case = st.fixed_dictionaries({
    "s": st.integers(1, 500),
    "skv": st.integers(1, 600),
    "hkv": st.integers(1, 2),
    "g": st.sampled_from([1, 4, 5, 8]),
    "p": st.sampled_from([0.0, 0.3, 1.0]),
    "seed": st.integers(0, 2 ** 16),
})


@settings(max_examples=40, **SETTINGS)
@given(c=bounds_case)
def test_forward_arbitrary_bounds_property(c):
    """Caller metadata may hold any key bounds (the reference validates only
    their shapes, V:360-383): half the rows get a sensible [start, end), the
    others random values from below 0 to past the last key, inverted or not,
    in no order.  Bounds are clipped to [0, keys); an empty or inverted range
    is an empty row (NaN / -inf), as in the oracle."""
    s, skv, hkv = c["s"], c["skv"], c["hkv"]
    hq = c["g"] * hkv
    rng = np.random.default_rng(c["seed"])
    gen = torch.Generator().manual_seed(c["seed"])
    q, k, v = workloads.make_qkv(gen, 1, s, skv, hq, hkv, 128)
    mask = torch.rand((1, s), generator=gen) < c["p"]
    ce = rng.integers(-20, skv + 20, s)
    fs, ls = rng.integers(-20, skv + 20, s), rng.integers(-20, skv + 20, s)
    sane = rng.random(s) < 0.5
    lo = rng.integers(0, skv, s)
    hi = np.minimum(lo + rng.integers(1, skv + 1, s), skv)
    fs, ce = np.where(sane, lo, fs), np.where(sane, hi, ce)
    ls = np.where(sane, np.maximum(lo, hi - rng.integers(1, 300, s)), ls)
    tag = f"bounds s{s} skv{skv} {hq}/{hkv} p{c['p']} seed{c['seed']}"
    print(f"[property] {tag}", flush=True)
    full, local = build_switch_query_indices(mask.to(DEV))
    o, lse = switch_gqa_prefill_forward(q.to(DEV), k.to(DEV), v.to(DEV), full, local,
                                        metadata=_metadata(fs, ls, ce, s, skv))
    torch.cuda.synchronize()
    f_np, l_np = R.compact(mask.numpy())
    o_ref, lse_ref = oracle.routed_attention(
        q, k, v, f_np, l_np, metadata={"full_starts": fs, "local_starts": ls, "causal_ends": ce})
    _assert_close(o, lse, o_ref, lse_ref, tag=tag)


@settings(max_examples=20, **SETTINGS)
@given(c=bounds_case)
def test_backward_monotone_bounds_property(c):
    """The backward takes any caller metadata whose key bounds do not
    decrease along each list (starts past their end count as the end):
    random sorted bounds, some rows empty, against the oracle."""
    s, skv, hkv = c["s"], c["skv"], c["hkv"]
    hq = c["g"] * hkv
    rng = np.random.default_rng(c["seed"])
    gen = torch.Generator().manual_seed(c["seed"])
    q, k, v = workloads.make_qkv(gen, 1, s, skv, hq, hkv, 128)
    mask = torch.rand((1, s), generator=gen) < c["p"]
    do = torch.randn(q.shape, generator=gen).to(torch.bfloat16)
    ce = np.sort(rng.integers(-5, skv + 5, s))
    fs = np.maximum.accumulate(np.minimum(np.sort(rng.integers(-5, skv + 5, s)),
                                          ce + rng.integers(0, 3, s)))
    ls = np.maximum.accumulate(np.minimum(np.sort(rng.integers(-5, skv + 5, s)),
                                          ce + rng.integers(0, 3, s)))
    tag = f"monotone bounds s{s} skv{skv} {hq}/{hkv} p{c['p']} seed{c['seed']}"
    print(f"[property] {tag}", flush=True)
    md = _metadata(fs, ls, ce, s, skv)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    full, local = build_switch_query_indices(mask.to(DEV))
    o, lse = switch_gqa_prefill_forward(qd, kd, vd, full, local, metadata=md)
    grads = switch_gqa_prefill_backward(qd, kd, vd, o, lse, do.to(DEV), full, local, metadata=md)
    torch.cuda.synchronize()
    f_np, l_np = R.compact(mask.numpy())
    refs = oracle.routed_attention_backward(
        q, k, v, do, f_np, l_np,
        metadata={"full_starts": fs, "local_starts": ls, "causal_ends": ce}, out=o.cpu())
    for name, g, r in zip(("dq", "dk", "dv"), grads, refs):
        _grad_close(g, r, f"{tag} {name}")


split_case = st.fixed_dictionaries({
    "b": st.integers(1, 2),
    "s": st.integers(520, 1800),
    "dkv": st.integers(-300, 300),
    "hkv": st.integers(1, 2),
    "g": st.sampled_from([1, 2, 4, 8]),
    "w": st.integers(1, 1500),
    "p": st.sampled_from([0.05, 0.3, 0.7, 1.0]),
    "seed": st.integers(0, 2 ** 16),
})


@settings(max_examples=25, **SETTINGS)
@given(c=split_case)
def test_split_paths_property(c):
    """Few KV heads and sequences of 9-29 key tiles: grids of a few dozen
    row tiles, where the forward cuts full items into key chunks of 4-32
    tiles (merged by their LSE) and the backward cuts long dQ row tiles into
    pieces (summed in order).  The forward against the oracle and against
    the unsplit C-ABI call (plain workspace), the backward against the
    oracle."""
    from switchattentionkernels_amd import _lib
    skv = max(1, c["s"] + c["dkv"])
    hq = c["g"] * c["hkv"]
    gen = torch.Generator().manual_seed(c["seed"])
    q, k, v = workloads.make_qkv(gen, c["b"], c["s"], skv, hq, c["hkv"], 128)
    mask = torch.rand((c["b"], c["s"]), generator=gen) < c["p"]
    do = torch.randn(q.shape, generator=gen).to(torch.bfloat16)
    L = _lib.lib()
    f_np, l_np = R.compact(mask.numpy())
    plain = L.swattn_prefill_workspace_bytes(c["b"], skv, c["hkv"], 128)
    split = L.swattn_prefill_split_workspace_bytes(c["b"], c["s"], skv, hq, c["hkv"], 128,
                                                   c["w"], f_np.size, l_np.size)
    tag = (f"split b{c['b']} s{c['s']} skv{skv} {hq}/{c['hkv']} w{c['w']} p{c['p']} "
           f"seed{c['seed']} fwd split {split > plain}")
    print(f"[property] {tag}", flush=True)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    full, local = build_switch_query_indices(mask.to(DEV))
    o, lse = switch_gqa_prefill_forward(qd, kd, vd, full, local, window_size=c["w"])
    grads = switch_gqa_prefill_backward(qd, kd, vd, o, lse, do.to(DEV), full, local,
                                        window_size=c["w"])
    ws = torch.empty(plain, dtype=torch.uint8, device=DEV)
    o_u, lse_u = torch.empty_like(qd), torch.empty(q.shape[:3], dtype=torch.float32, device=DEV)
    st_ = L.swattn_prefill_fwd(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), full.data_ptr(),
                               full.numel(), local.data_ptr(), local.numel(), None, None, None,
                               o_u.data_ptr(), lse_u.data_ptr(), c["b"], c["s"], skv, hq,
                               c["hkv"], 128, c["w"], 128 ** -0.5 * oracle.LOG2E, ws.data_ptr(),
                               plain, _lib.stream_handle(qd.device))
    assert st_ == 0, L.swattn_last_error()
    torch.cuda.synchronize()
    o_ref, lse_ref = oracle.routed_attention(q, k, v, f_np, l_np, window_size=c["w"])
    _assert_close(o, lse, o_ref, lse_ref, tag=tag)
    _assert_close(o, lse, o_u.float().cpu(), lse_u.cpu(), tag=tag + " vs unsplit")
    refs = oracle.routed_attention_backward(q, k, v, do, f_np, l_np, window_size=c["w"],
                                            out=o.cpu())
    for name, g, r in zip(("dq", "dk", "dv"), grads, refs):
        _grad_close(g, r, f"{tag} {name}")
