"""GPU parity of the routed prefill backward (dq, dk, dv) against the oracle.

The reference is forward-only (V:14-15); the oracle's backward is the
derivative of its pinned forward (see tests/test_oracle.py for its pins).

Bar, per gradient tensor, against the fp32 oracle on the same bf16 inputs:
* relative L2 error ||g - g_ref|| / ||g_ref|| <= 1e-2;
* max-abs error <= 3e-2 * max|g_ref|.
The kernel rounds P and dS to bf16 for the products and writes bf16 results
(2^-9 relative each), and takes Delta = dO . O from the bf16 forward output;
those errors are a few 1e-3 in both measures, and a wrong index, sign or
dropped term gives errors of order 1.
Full-size configs are checked on sampled rows (dq) plus the size-independent
identities sum_j dk_j = 0 and sum_j dv_j = sum of the group's dO rows.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle import routing as R
from switchattentionkernels_amd import (
    build_switch_attention_metadata,
    build_switch_query_indices,
    shard_attention_metadata,
    switch_gqa_prefill,
    switch_gqa_prefill_backward,
    switch_gqa_prefill_forward,
    switch_gqa_prefill_varlen,
    switch_gqa_prefill_varlen_forward,
    workloads,
)
from switchattentionkernels_amd.metadata import SwitchAttentionMetadata

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL_L2, REL_MAX = 1e-2, 3e-2


def _qkv(seed, b, s, hq, hkv, skv=None):
    gen = torch.Generator().manual_seed(seed)
    q, k, v = workloads.make_qkv(gen, b, s, s if skv is None else skv, hq, hkv, 128)
    do = torch.randn(b, s, hq, 128, generator=gen).to(torch.bfloat16)
    return q, k, v, do


def _mask(seed, shape, p):
    return torch.rand(shape, generator=torch.Generator().manual_seed(seed + 11)) < p


def _grad_close(got, ref, tag, rows=None):
    got = got.float().cpu()
    ref = ref.float()
    if rows is not None:
        got, ref = got.reshape(-1, *got.shape[2:])[rows], ref.reshape(-1, *ref.shape[2:])[rows]
    assert torch.isfinite(got).all(), f"{tag}: non-finite gradient"
    err = got - ref
    l2 = float(err.norm() / ref.norm().clamp_min(1e-20))
    mx = float(err.abs().max() / ref.abs().max().clamp_min(1e-20))
    print(f"[grad] {tag}: rel_l2 {l2:.2e} rel_max {mx:.2e}", flush=True)
    assert l2 <= REL_L2 and mx <= REL_MAX, f"{tag}: rel_l2 {l2:.3e} rel_max {mx:.3e}"


def _run(q, k, v, do, mask, window, metadata=None, md_np=None, sm_scale=None):
    full, local = build_switch_query_indices(mask.to(DEV))
    qd, kd, vd, dod = q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV)
    o, lse = switch_gqa_prefill_forward(qd, kd, vd, full, local, window_size=window,
                                        metadata=metadata, sm_scale=sm_scale)
    dq, dk, dv = switch_gqa_prefill_backward(qd, kd, vd, o, lse, dod, full, local,
                                             window_size=window, metadata=metadata,
                                             sm_scale=sm_scale)
    torch.cuda.synchronize()
    return dq, dk, dv


def _oracle(q, k, v, do, mask, window, md_np=None, rows=None, sm_scale=None):
    full, local = R.compact(mask.numpy())
    return oracle.routed_attention_backward(q, k, v, do, full, local, window_size=window,
                                            metadata=md_np, rows=rows, sm_scale=sm_scale)


def _md_np(md):
    return {n: getattr(md, n).cpu().numpy() for n in ("full_starts", "local_starts",
                                                      "causal_ends")}


@pytest.mark.parametrize("b,s,hq,hkv,w,p,skv", [
    (1, 300, 8, 2, 64, 0.3, None),      # G = 4, ragged length
    (2, 257, 4, 4, 100, 0.5, None),     # G = 1, two batch rows
    (1, 520, 40, 8, 128, 0.25, None),   # G = 5: blocks straddle query positions
    (1, 200, 64, 8, 1, 0.2, None),      # G = 8, window 1
    (1, 1000, 32, 8, 1024, 0.25, None), # window beyond the sequence
    (1, 384, 8, 2, 96, 0.0, None),      # all local
    (1, 384, 8, 2, 96, 1.0, None),      # all full (dense causal)
    (1, 300, 8, 2, 64, 0.4, 180),       # fewer keys than queries
    (2, 200, 8, 2, 50, 0.3, 333),       # more keys than queries
    (3, 512, 8, 2, 100, 0.3, None),     # whole 256-key tiles per sequence: interleaved
                                        # dK/dV pair order, 12 pairs split 16 ways
    (3, 164, 8, 1, 2, 0.3, 3),          # seq_q > seq_kv + W - 1: late local rows have
    (2, 300, 8, 2, 64, 0.3, 100),       # empty ranges starting past the next sequence's
                                        # first start (the block search must still find it)
])
def test_backward_matches_oracle(b, s, hq, hkv, w, p, skv):
    q, k, v, do = _qkv(b * 1000 + s, b, s, hq, hkv, skv)
    m = _mask(s + hq, (b, s), p)
    dq, dk, dv = _run(q, k, v, do, m, w)
    rq, rk, rv = _oracle(q, k, v, do, m, w)
    tag = f"b{b} s{s} {hq}/{hkv} w{w} p{p} skv{skv}"
    _grad_close(dq, rq, tag + " dq")
    _grad_close(dk, rk, tag + " dk")
    _grad_close(dv, rv, tag + " dv")


def test_backward_custom_scale_and_determinism():
    q, k, v, do = _qkv(5, 1, 400, 16, 4)
    m = _mask(5, (1, 400), 0.3)
    a = _run(q, k, v, do, m, 77, sm_scale=0.03)
    bb = _run(q, k, v, do, m, 77, sm_scale=0.03)
    for x, y in zip(a, bb):
        assert torch.equal(x, y)   # no atomics: bit-identical reruns
    ref = _oracle(q, k, v, do, m, 77, sm_scale=0.03)
    for g, r, n in zip(a, ref, ("dq", "dk", "dv")):
        _grad_close(g, r, "sm_scale=0.03 " + n)


def test_backward_varlen_metadata():
    cu = [0, 300, 301, 700, 1100]
    q, k, v, do = _qkv(9, 1, 1100, 16, 4)
    m = _mask(9, (1, 1100), 0.3)
    md = build_switch_attention_metadata(1100, 1100, device=DEV, window_size=128, cu_seqlens=cu)
    dq, dk, dv = _run(q, k, v, do, m, 128, metadata=md)
    ref = _oracle(q, k, v, do, m, 128, md_np=_md_np(md))
    for g, r, n in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
        _grad_close(g, r, "varlen " + n)


def test_backward_key_chunk_with_empty_rows():
    """Query rows 512..767 of a 1024-token sequence against the key chunk
    [600, 1000): rows before 600 see no key there (dq = 0) and keys no row
    can see get dk = dv = 0."""
    s, hq, hkv, w = 1024, 8, 2, 64
    q, k, v, do = _qkv(13, 1, s, hq, hkv)
    m = _mask(13, (1, s), 0.3)
    rows = torch.arange(512, 768, dtype=torch.int32)
    md = shard_attention_metadata(rows.to(DEV), kv_start=600, kv_end=1000, window_size=w)
    qs, dos, ms = q[:, 512:768].contiguous(), do[:, 512:768].contiguous(), m[:, 512:768]
    kc, vc = k[:, 600:1000].contiguous(), v[:, 600:1000].contiguous()
    dq, dk, dv = _run(qs, kc, vc, dos, ms, w, metadata=md)
    ref = _oracle(qs, kc, vc, dos, ms, w, md_np=_md_np(md))
    assert torch.count_nonzero(dq[0, :600 - 512].float()) == 0
    assert torch.count_nonzero(dk[0, 768 - 600:].float()) == 0
    for g, r, n in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
        _grad_close(g, r, "chunk " + n)


def test_autograd_function_matches_backward():
    q, k, v, do = _qkv(17, 1, 333, 8, 2)
    m = _mask(17, (1, 333), 0.25)
    full, local = build_switch_query_indices(m.to(DEV))
    qd, kd, vd = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
    out, lse = switch_gqa_prefill(qd, kd, vd, full, local, window_size=40)
    assert not lse.requires_grad
    (out.float() * do.to(DEV).float()).sum().backward()
    dq, dk, dv = _run(q, k, v, do, m, 40)
    assert torch.equal(qd.grad, dq) and torch.equal(kd.grad, dk) and torch.equal(vd.grad, dv)


def test_varlen_autograd_matches_oracle():
    cu = [0, 200, 201, 640]
    q, k, v, do = _qkv(21, 1, 640, 8, 2)
    m = _mask(21, (1, 640), 0.3)
    full, local = build_switch_query_indices(m.to(DEV))
    qd, kd, vd = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
    out, _ = switch_gqa_prefill_varlen(qd, kd, vd, full, local, cu, window_size=64)
    (out.float() * do.to(DEV).float()).sum().backward()
    md = build_switch_attention_metadata(640, 640, device=DEV, window_size=64, cu_seqlens=cu)
    ref = _oracle(q, k, v, do, m, 64, md_np=_md_np(md))
    for g, r, n in zip((qd.grad, kd.grad, vd.grad), ref, ("dq", "dk", "dv")):
        _grad_close(g, r, "varlen autograd " + n)


def test_backward_rejects_non_monotone_metadata():
    """The backward locates the rows that see a key block by binary search over
    each list's bounds, so metadata whose bounds go down along a list is refused
    (the forward accepts it)."""
    s = 64
    q, k, v, do = _qkv(23, 1, s, 4, 2)
    m = torch.zeros(1, s, dtype=torch.bool)
    md = build_switch_attention_metadata(s, s, device=DEV, window_size=16)
    ends = md.causal_ends.clone()
    ends[10] = 3   # row 10 now ends before row 9
    bad = SwitchAttentionMetadata(md.q_positions, md.kv_positions, md.q_segment_ids,
                                  md.kv_segment_ids, md.full_starts, md.local_starts, ends)
    full, local = build_switch_query_indices(m.to(DEV))
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = switch_gqa_prefill_forward(qd, kd, vd, full, local, window_size=16, metadata=bad)
    with pytest.raises(ValueError, match="non-decreasing"):
        switch_gqa_prefill_backward(qd, kd, vd, o, lse, do.to(DEV), full, local, window_size=16,
                                    metadata=bad)


def test_b2_config_backward():
    wl = workloads.build("b2", seed=3, p_full=0.25)
    gen = torch.Generator().manual_seed(4)
    do = torch.randn(wl["q"].shape, generator=gen).to(torch.bfloat16)
    dq, dk, dv = _run(wl["q"], wl["k"], wl["v"], do, wl["mask"], wl["window"])
    ref = _oracle(wl["q"], wl["k"], wl["v"], do, wl["mask"], wl["window"])
    for g, r, n in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
        _grad_close(g, r, "config b2 " + n)


def test_s16k_backward_identities_and_sampled_rows():
    wl = workloads.build("s16k", seed=0)
    q, k, v, m, w = wl["q"], wl["k"], wl["v"], wl["mask"], wl["window"]
    gen = torch.Generator().manual_seed(5)
    do = torch.randn(q.shape, generator=gen).to(torch.bfloat16)
    dq, dk, dv = _run(q, k, v, do, m, w)
    s, hq, hkv = q.shape[1], q.shape[2], k.shape[2]
    g = hq // hkv
    # sum_j dk_j = 0 per KV head (softmax is shift invariant in the keys),
    # up to the bf16 rounding of each dk row.
    dk32 = dk[0].float()
    assert (dk32.sum(0).abs() <= 2e-3 * dk32.abs().sum(0) + 1e-3).all()
    # sum_j dv_j = sum of dO over the group's query rows (rows of P sum to 1).
    dv_sum = dv[0].float().sum(0).cpu()
    ref = do[0].float().reshape(s, hkv, g, 128).sum((0, 2))
    assert ((dv_sum - ref).abs() <= 2e-3 * do[0].float().abs().reshape(s, hkv, g, 128)
            .sum((0, 2)) + 1e-2).all()
    rows = np.unique(np.concatenate([np.random.default_rng(0).choice(s, 384, replace=False),
                                     [0, 1, 1023, 1024, s - 1]]))
    rq, _, _ = _oracle(q, k, v, do, m, w, rows=rows)
    _grad_close(dq, rq, "s16k dq sampled rows", rows=torch.as_tensor(rows))


@pytest.mark.parametrize("b,s,hq,hkv,w,p", [
    (1, 4096, 4, 1, 256, 0.3),    # dQ pieces of 4 key tiles: full row tiles in up to 17,
                                  # local ones (6 tiles) in 2
    (2, 2000, 8, 1, 700, 0.6),    # two sequences, pieces of 8: full in up to 5, local in 2
])
def test_backward_dq_pieces_match_oracle(b, s, hq, hkv, w, p):
    """Few row tiles (one KV head): the longest dQ row tiles are cut into
    pieces whose fp32 partials are summed in piece order."""
    q, k, v, do = _qkv(b * 77 + s, b, s, hq, hkv)
    m = _mask(s + 7, (b, s), p)
    dq, dk, dv = _run(q, k, v, do, m, w)
    rq, rk, rv = _oracle(q, k, v, do, m, w)
    tag = f"pieces b{b} s{s} {hq}/{hkv} w{w} p{p}"
    _grad_close(dq, rq, tag + " dq")
    _grad_close(dk, rk, tag + " dk")
    _grad_close(dv, rv, tag + " dv")
    # the latest full rows see every earlier key: their row tiles are cut the most
    f_np, _ = R.compact(m.numpy())
    late = torch.as_tensor(f_np[-64:])
    _grad_close(dq, rq, tag + " dq late full rows", rows=late)


def test_kv_head_share_backward():
    """One GPU's share of config #3 under a KV-head split (Hq4/Hkv1, S=16384,
    W1024, p_full 0.25): dQ row tiles are cut into pieces.  Sampled dq rows
    (late full rows included) against the oracle, dk / dv by the identities
    of the config #3 test."""
    wl = workloads.build("kvh1", seed=2)
    q, k, v, m, w = wl["q"], wl["k"], wl["v"], wl["mask"], wl["window"]
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    dq, dk, dv = _run(q, k, v, do, m, w)
    s, hq, hkv = q.shape[1], q.shape[2], k.shape[2]
    g = hq // hkv
    dk32 = dk[0].float()
    assert (dk32.sum(0).abs() <= 2e-3 * dk32.abs().sum(0) + 1e-3).all()
    dv_sum = dv[0].float().sum(0).cpu()
    ref = do[0].float().reshape(s, hkv, g, 128).sum((0, 2))
    assert ((dv_sum - ref).abs() <= 2e-3 * do[0].float().abs().reshape(s, hkv, g, 128)
            .sum((0, 2)) + 1e-2).all()
    f_np, _ = R.compact(m.numpy())
    rows = np.unique(np.concatenate([np.random.default_rng(2).choice(s, 256, replace=False),
                                     f_np[-96:], [0, s - 1]]))
    rq, _, _ = _oracle(q, k, v, do, m, w, rows=rows)
    _grad_close(dq, rq, "kvh1 dq sampled rows", rows=torch.as_tensor(rows))


@pytest.mark.parametrize("b,s,hq,hkv,w,p,skv", [
    (1, 300, 8, 2, 64, 0.3, None),      # dQ row tiles cut into pieces
    (2, 300, 8, 2, 64, 0.3, 100),       # fewer keys than queries: rows with no key (dq = 0)
    (1, 4096, 4, 1, 256, 0.3, None),    # pieces of 4 tiles, full and local row tiles cut
    (1, 2000, 32, 8, 1024, 0.25, None), # no pieces
])
def test_backward_writes_every_dq_row(b, s, hq, hkv, w, p, skv):
    """Through the C ABI with dq, dk and dv pre-filled with NaN: lists that
    cover every position get every dq row written (0 for a row with no key),
    and every dk / dv row, so the Python layer allocates them uninitialised."""
    from switchattentionkernels_amd import _lib
    q, k, v, do = _qkv(b * 31 + s, b, s, hq, hkv, skv)
    m = _mask(s + 3, (b, s), p)
    qd, kd, vd, dod = q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV)
    full, local = build_switch_query_indices(m.to(DEV))
    o, lse = switch_gqa_prefill_forward(qd, kd, vd, full, local, window_size=w)
    L = _lib.lib()
    skv_ = k.shape[1]
    ws_bytes = L.swattn_prefill_bwd_workspace_bytes(b, skv_, hq, hkv, 128, w, full.numel(),
                                                    local.numel())
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    dq = torch.full_like(qd, float("nan"))
    dk = torch.full_like(kd, float("nan"))
    dv = torch.full_like(vd, float("nan"))
    st = L.swattn_prefill_bwd(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o.data_ptr(),
                              lse.data_ptr(), dod.data_ptr(), full.data_ptr(), full.numel(),
                              local.data_ptr(), local.numel(), None, None, None, dq.data_ptr(),
                              dk.data_ptr(), dv.data_ptr(), b, s, skv_, hq, hkv, 128, w,
                              128 ** -0.5 * oracle.LOG2E, ws.data_ptr(), ws_bytes,
                              _lib.stream_handle(qd.device))
    assert st == 0, L.swattn_last_error()
    torch.cuda.synchronize()
    for name, g in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.isfinite(g).all().item(), f"{name}: a row was never written"
    rq, rk, rv = _oracle(q, k, v, do, m, w)
    tag = f"NaN canary b{b} s{s} {hq}/{hkv} w{w} skv{skv}"
    _grad_close(dq, rq, tag + " dq")
    _grad_close(dk, rk, tag + " dk")
    _grad_close(dv, rv, tag + " dv")


@pytest.mark.parametrize("qk_scale", [4.0, 0.05])
def test_backward_peaked_and_flat_softmax(qk_scale):
    """Gradients when rows are nearly one-hot (Q, K x4) or nearly uniform
    (Q, K x0.05), against the oracle."""
    q, k, v, do = _qkv(23, 1, 600, 8, 2)
    q, k = (q.float() * qk_scale).to(torch.bfloat16), (k.float() * qk_scale).to(torch.bfloat16)
    m = _mask(23, (1, 600), 0.4)
    dq, dk, dv = _run(q, k, v, do, m, 150)
    rq, rk, rv = _oracle(q, k, v, do, m, 150)
    tag = f"q,k x{qk_scale}"
    _grad_close(dq, rq, tag + " dq")
    _grad_close(dk, rk, tag + " dk")
    _grad_close(dv, rv, tag + " dv")


def test_backward_with_no_query_rows():
    """No query rows: dq is empty and every key gets dk = dv = 0."""
    q = torch.zeros(1, 0, 4, 128, dtype=torch.bfloat16, device=DEV)
    k = torch.randn(1, 70, 2, 128, device=DEV).to(torch.bfloat16)
    v = torch.randn(1, 70, 2, 128, device=DEV).to(torch.bfloat16)
    full, local = build_switch_query_indices(torch.zeros(1, 0, dtype=torch.bool, device=DEV))
    o, lse = switch_gqa_prefill_forward(q, k, v, full, local, window_size=8)
    dq, dk, dv = switch_gqa_prefill_backward(q, k, v, o, lse, torch.zeros_like(q), full, local,
                                             window_size=8)
    torch.cuda.synchronize()
    assert dq.shape == q.shape
    assert torch.count_nonzero(dk) == 0 and torch.count_nonzero(dv) == 0


def test_backward_few_key_rows_delta_convention():
    """Regression (found by a randomized sweep): two packed rows, cu_seqlens
    [0, 2], Hq = Hkv = 1, window 2, every row local, seed 0 -- row 0 sees
    one key, row 1 two.  The kernel takes Delta = dO . O from the bf16
    forward output (the FlashAttention-2 convention), which moves dq of the
    two-key row by 1.3-1.5e-2 relative L2 against the exact gradient: above
    the plain 1e-2 bar, by a shift that is known exactly.

    * Against the oracle with the same convention (Delta from the kernel's
      own O), every gradient meets the plain bar.
    * Against the exact gradient, each dq row lies within its Delta shift
      scale * |dO . (O_bf16 - O)| * ||sum_j P_rj k_j|| (10 % slack) plus
      1e-2 of its own norm plus a floor of 1e-2 of the rms row norm; the
      CPU test ``test_delta_convention_shift_is_the_bound`` shows a dropped
      or doubled Delta breaks that bound on this input."""
    from test_oracle import _delta_bound_excess, _few_key_case
    q, k, v, do, full_np, local_np, md_np = _few_key_case()
    cu = [0, 2]
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    mask = torch.zeros(1, 2, dtype=torch.bool)
    full, local = build_switch_query_indices(mask.to(DEV))
    o, lse = switch_gqa_prefill_varlen_forward(qd, kd, vd, full, local, cu, window_size=2)
    md = build_switch_attention_metadata(2, 2, device=DEV, window_size=2, cu_seqlens=cu)
    dq, dk, dv = switch_gqa_prefill_backward(qd, kd, vd, o, lse, do.to(DEV), full, local,
                                             metadata=md, window_size=2)
    torch.cuda.synchronize()
    o_cpu = o.cpu()
    conv = oracle.routed_attention_backward(q, k, v, do, full_np, local_np, metadata=md_np,
                                            out=o_cpu)
    for name, g, r in zip(("dq", "dk", "dv"), (dq, dk, dv), conv):
        _grad_close(g, r, f"few-key {name} vs Delta-convention oracle")
    terms = {}
    exact = oracle.routed_attention_backward(q, k, v, do, full_np, local_np, metadata=md_np,
                                             delta_terms=terms)
    o_exact, _ = oracle.routed_attention(q, k, v, full_np, local_np, metadata=md_np)
    rel = float((dq.float().cpu() - exact[0]).norm() / exact[0].norm())
    excess = _delta_bound_excess(dq.float().cpu(), exact[0], o_cpu, o_exact, do, terms)
    print(f"[grad] few-key dq vs exact: rel_l2 {rel:.3e}, bound excess {excess:.3e}", flush=True)
    assert excess <= 0, f"dq row outside its Delta-convention bound by {excess:.3e}"
