"""The forward's key-range split of long full items (few KV heads, long
sequences), against the oracle and against the unsplit kernel.

swattn_prefill_fwd splits full items into chunks of 4 to 64 key tiles (at
fixed multiples of the chunk size) when the longest one would set the
kernel's length and the caller passes the workspace that
swattn_prefill_split_workspace_bytes() asks for; the chunks are merged by
their log2 LSE (V:236-241).  Checked here:

* parity with the oracle on sampled rows, late causal rows (the split ones)
  included, at the usual bars (O max-abs <= 2e-2, mean-abs <= 2e-3, LSE
  relative <= 1e-3), and every routed row written (NaN canary);
* split against unsplit (the same call with the smaller workspace): equal to
  rounding, and bit-identical on the items that lie inside one chunk;
* an item whose rows span more chunks than it has slots (a sparse full list
  over several sequences) runs whole.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle
from oracle import routing as R
from switchattentionkernels_amd import (build_switch_query_indices, switch_gqa_prefill_forward,
                                        workloads)
from switchattentionkernels_amd import _lib

from test_gpu_parity import _assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _abi_forward(q, k, v, full, local, window, split):
    """swattn_prefill_fwd through the C ABI with the split (or the plain)
    workspace; O and LSE pre-filled with NaN."""
    b, s, hq, _ = q.shape
    skv, hkv = k.shape[1], k.shape[2]
    L = _lib.lib()
    base = L.swattn_prefill_workspace_bytes(b, skv, hkv, 128)
    big = L.swattn_prefill_split_workspace_bytes(b, s, skv, hq, hkv, 128, window, full.numel(),
                                                 local.numel())
    ws_bytes = big if split else base
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    out = torch.full_like(q, float("nan"))
    lse = torch.full(q.shape[:3], float("nan"), device=DEV)
    st = L.swattn_prefill_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), full.data_ptr(),
                              full.numel(), local.data_ptr(), local.numel(), None, None, None,
                              out.data_ptr(), lse.data_ptr(), b, s, skv, hq, hkv, 128, window,
                              ctypes.c_float(128 ** -0.5 * oracle.LOG2E), ws.data_ptr(), ws_bytes,
                              _lib.stream_handle(q.device))
    assert st == 0, L.swattn_last_error()
    torch.cuda.synchronize()
    return out, lse, base, big


def _split_tiles(s, hq, hkv, w, n_full, n_local):
    """The chunk size (64-key tiles) of the library's split plan: 1.5 times
    the estimated key tiles per workgroup slot (full items at half a
    sequence, local ones at their window, over 512 slots), clamped to
    [4, 64], and at least what keeps the chunk slots (full items x KV heads x
    sequence tiles / chunk) under 2048.  Used only to pick the rows that must
    come out bit-identical; a wrong value here would fail the equality
    below."""
    g = hq // hkv
    full_items, local_items = -(-n_full * g // 128), -(-n_local * g // 128)
    seq_tiles = -(-s // 64)
    local_tiles = -(-min(w, s) // 64) + 2
    est = hkv * (full_items * (seq_tiles // 2 + 2) + local_items * local_tiles)
    chunk = min(64, max(4, (3 * (est // 512)) // 2))
    return max(chunk, -(-full_items * hkv * seq_tiles // 2048))


def _case(seed, b, s, hq, hkv, p):
    gen = torch.Generator().manual_seed(seed)
    q, k, v = workloads.make_qkv(gen, b, s, s, hq, hkv, 128)
    mask = torch.rand((b, s), generator=gen) < p
    return q, k, v, mask


@pytest.mark.parametrize("b,s,hq,hkv,w,p", [
    (1, 8192, 4, 1, 1024, 0.25),    # longest full item 129 tiles: chunks of 22 tiles
    (2, 6000, 2, 1, 300, 0.5),      # two sequences, chunks of 15 tiles: items inside one
                                    # chunk and across several
    (1, 1024, 8, 2, 256, 0.25),     # config #1's shape: about 64 items on 256 CUs, chunks
                                    # of 4 tiles
])
def test_split_matches_oracle_and_unsplit(b, s, hq, hkv, w, p):
    q, k, v, mask = _case(31 + s, b, s, hq, hkv, p)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    full, local = build_switch_query_indices(mask.to(DEV))
    o_s, l_s, base, big = _abi_forward(qd, kd, vd, full, local, w, split=True)
    assert big > base, "this shape must take the split"
    print(f"split b{b} s{s} {hq}/{hkv}: workspace {base} -> {big}", flush=True)
    assert not torch.isnan(o_s).any() and not torch.isnan(l_s).any(), "a row was never written"
    o_u, l_u, _, _ = _abi_forward(qd, kd, vd, full, local, w, split=False)
    # rows of full items that lie inside one chunk, and every local row, are
    # computed exactly as unsplit; late causal rows differ by rounding only
    f_np, l_np = R.compact(mask.numpy())
    # A full item (128 rows = 128 / G listed positions, head fastest) lies inside one
    # chunk when its rows' keys [b*s, b*s + i + 1), in flattened key coordinates, start
    # and end in the same chunk, counted as the kernel counts them.
    one_chunk = np.ones(b * s, dtype=bool)
    g = hq // hkv
    ct = _split_tiles(s, hq, hkv, w, f_np.size, l_np.size)
    for it in range(-(-f_np.size * g // 128)):
        sl = f_np[(128 * it) // g:min((128 * it + 127) // g, f_np.size - 1) + 1]
        lo, hi = int((sl // s * s).min()), int((sl // s * s + sl % s + 1).max())
        c0, c1 = (lo // 64) // ct, ((hi + 63) // 64 - 1) // ct
        one_chunk[sl] = c0 == c1
    ok = torch.as_tensor(one_chunk)
    assert ok.any() and not ok.all()
    o_s_c, o_u_c = o_s.reshape(b * s, hq, 128).cpu(), o_u.reshape(b * s, hq, 128).cpu()
    assert torch.equal(o_s_c[ok], o_u_c[ok])
    assert torch.equal(l_s.reshape(b * s, hq).cpu()[ok], l_u.reshape(b * s, hq).cpu()[ok])
    _assert_close(o_s, l_s, o_u.float().cpu(), l_u.cpu(), tag="split vs unsplit")
    rng = np.random.default_rng(s)
    rows = np.unique(np.concatenate([rng.integers(0, b * s, 300),
                                     f_np[-64:], np.array([0, b * s - 1])]))
    o_r, l_r = oracle.routed_attention(q, k, v, f_np, l_np, window_size=w, rows=rows)
    _assert_close(o_s, l_s, o_r, l_r, rows=rows, tag=f"split b{b} s{s} vs oracle")


def test_items_spanning_many_sequences_run_whole():
    """A sparse full list over eight sequences: a 128-row item then holds
    rows of several sequences, its key range spans more chunks than it has
    slots, and it runs unsplit in one workgroup."""
    b, s, hq, hkv, w = 8, 4096, 4, 1, 256
    q, k, v, _ = _case(77, b, s, hq, hkv, 0.0)
    mask = torch.zeros(b, s, dtype=torch.bool)
    mask[:, -3:] = True                                      # 3 full rows per sequence
    mask[:, 100] = True
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    full, local = build_switch_query_indices(mask.to(DEV))
    o_s, l_s, base, big = _abi_forward(qd, kd, vd, full, local, w, split=True)
    print(f"sparse full list: workspace {base} -> {big}", flush=True)
    assert big > base   # the split runs: the item is whole inside a split launch
    assert not torch.isnan(o_s).any() and not torch.isnan(l_s).any()
    f_np, l_np = R.compact(mask.numpy())
    rows = np.unique(np.concatenate([f_np, np.arange(0, b * s, 97)]))
    o_r, l_r = oracle.routed_attention(q, k, v, f_np, l_np, window_size=w, rows=rows)
    _assert_close(o_s, l_s, o_r, l_r, rows=rows, tag="sparse full list vs oracle")


def test_kv_head_share_of_s16k():
    """One GPU's share of config #3 under a KV-head split (Hq4/Hkv1, S=16384,
    W1024, p_full 0.25) through the public API, which passes the split
    workspace: every row written, sampled rows against the oracle."""
    wl = workloads.build("kvh1", seed=3)
    q, k, v, m = wl["q"], wl["k"], wl["v"], wl["mask"]
    full, local = build_switch_query_indices(m.to(DEV))
    o, lse = switch_gqa_prefill_forward(q.to(DEV), k.to(DEV), v.to(DEV), full, local,
                                        window_size=wl["window"])
    torch.cuda.synchronize()
    # rows the kernel never wrote would hold whatever torch.empty gave: compare all
    # against NaN-free expectations on a sample, and check no NaN anywhere
    assert not torch.isnan(o).any() and torch.isfinite(lse).all()
    f_np, l_np = R.compact(m.numpy())
    rng = np.random.default_rng(3)
    rows = np.unique(np.concatenate([rng.integers(0, 16384, 200), f_np[-48:]]))
    o_r, l_r = oracle.routed_attention(q, k, v, f_np, l_np, window_size=wl["window"], rows=rows)
    _assert_close(o, lse, o_r, l_r, rows=rows, tag="kvh1 vs oracle")


def test_long_sparse_sequence_lengthens_the_chunks():
    """A 131072-key sequence with 2 % full rows (one KV head): chunks of 64
    tiles would need 33 slots per full item, so the plan lengthens them
    (about 2048 chunk slots in all) and the split workspace stays small.
    Sampled rows, late full rows included, against the oracle; no row left
    unwritten."""
    b, s, hq, hkv, w = 1, 131072, 4, 1, 1024
    gen = torch.Generator().manual_seed(41)
    q, k, v = workloads.make_qkv(gen, b, s, s, hq, hkv, 128)
    mask = torch.rand((b, s), generator=gen) < 0.02
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    full, local = build_switch_query_indices(mask.to(DEV))
    o, lse, base, big = _abi_forward(qd, kd, vd, full, local, w, split=True)
    assert base < big <= base + (200 << 20)
    print(f"long sparse: workspace {base} -> {big}", flush=True)
    assert not torch.isnan(o).any() and not torch.isnan(lse).any()
    f_np, l_np = R.compact(mask.numpy())
    rng = np.random.default_rng(41)
    rows = np.unique(np.concatenate([rng.integers(0, s, 100), f_np[-24:], f_np[:4]]))
    o_r, l_r = oracle.routed_attention(q, k, v, f_np, l_np, window_size=w, rows=rows)
    _assert_close(o, lse, o_r, l_r, rows=rows, tag="long sparse vs oracle")
