"""Pin the CPU oracle (CPU only).

Every oracle function is checked against something it does not share code
with: numpy/torch library routines, closed forms, a float64 brute force
written from the definitions, and invariants of the routing semantics.  The
last block plants mistakes in the oracle and checks that the pins catch them.
"""

import math

import numpy as np
import pytest
import torch

import oracle
from oracle import routing as R
from oracle import attention as A

# ----------------------------------------------------------------------------
# helpers
# ----------------------------------------------------------------------------


def _rand_qkv(seed, b, s, hq, hkv, d=128, skv=None, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    skv = s if skv is None else skv
    q = (torch.randn(b, s, hq, d, generator=g) * scale).to(torch.bfloat16)
    k = (torch.randn(b, skv, hkv, d, generator=g) * scale).to(torch.bfloat16)
    v = (torch.randn(b, skv, hkv, d, generator=g) * scale).to(torch.bfloat16)
    return q, k, v


def _mask(seed, shape, p):
    g = torch.Generator().manual_seed(seed + 1000)
    return torch.rand(shape, generator=g) < p


def _routed(q, k, v, mask, window, **kw):
    full, local = R.compact(mask.numpy())
    return A.routed_attention(q, k, v, full, local, window_size=window, **kw)


# ----------------------------------------------------------------------------
# compaction (V:306-322)
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("n,p", [(1, 0.5), (7, 0.0), (7, 1.0), (64, 0.5), (1000, 0.25),
                                 (4097, 0.9), (16385, 0.1)])
def test_compact_matches_nonzero(n, p):
    m = _mask(n, (n,), p)
    full, local = R.compact(m.numpy())
    assert full.dtype == np.int32 and local.dtype == np.int32
    np.testing.assert_array_equal(full, np.flatnonzero(m.numpy()))
    np.testing.assert_array_equal(local, np.flatnonzero(~m.numpy()))
    # the reference's own expression, torch boolean indexing on arange (V:321-322)
    pos = torch.arange(n, dtype=torch.int32)
    assert torch.equal(torch.from_numpy(full), pos[m])
    assert torch.equal(torch.from_numpy(local), pos[~m])


def test_compact_alternating_and_2d():
    m = (torch.arange(129) % 2 == 0)
    full, local = R.compact(m.numpy())
    np.testing.assert_array_equal(full, np.arange(0, 129, 2))
    np.testing.assert_array_equal(local, np.arange(1, 129, 2))
    m2 = _mask(3, (3, 50), 0.4)
    f2, l2 = R.compact(m2.numpy())
    np.testing.assert_array_equal(f2, np.flatnonzero(m2.numpy().reshape(-1)))
    np.testing.assert_array_equal(l2, np.flatnonzero(~m2.numpy().reshape(-1)))


# ----------------------------------------------------------------------------
# index checks (V:299-302, V:392-393)
# ----------------------------------------------------------------------------

def test_check_indices_each_condition():
    ok_f, ok_l = np.array([0, 3, 5]), np.array([1, 2, 4, 6])
    assert R.check_indices(ok_f, ok_l, 7) == 0
    assert R.first_error(ok_f, ok_l, 7) is None
    cases = [
        (np.array([0, 3, 7]), ok_l, R.ERR_FULL_RANGE, R.MSG_RANGE),
        (np.array([-1, 3, 5]), ok_l, R.ERR_FULL_RANGE, R.MSG_RANGE),
        (np.array([3, 0, 5]), ok_l, R.ERR_FULL_ORDER, R.MSG_ORDER),
        (np.array([0, 3, 3]), ok_l, R.ERR_FULL_ORDER, R.MSG_ORDER),
        (ok_f, np.array([1, 2, 4, 9]), R.ERR_LOCAL_RANGE, R.MSG_RANGE),
        (ok_f, np.array([2, 1, 4, 6]), R.ERR_LOCAL_ORDER, R.MSG_ORDER),
        (ok_f, np.array([1, 2, 3, 6]), R.ERR_OVERLAP, R.MSG_DISJOINT),
    ]
    for f, l, bit, msg in cases:
        assert R.check_indices(f, l, 7) == bit, (f, l)
        assert R.first_error(f, l, 7) == (ValueError, msg)
    # count-based coverage (V:392-393)
    assert R.first_error(ok_f, np.array([1, 2, 4]), 7) == (ValueError, R.MSG_COVER)
    # reference order: full-list errors win over local-list errors
    assert R.first_error(np.array([3, 0, 5]), np.array([9, 1, 2, 4]), 7) == (ValueError, R.MSG_ORDER)


# ----------------------------------------------------------------------------
# bounds and metadata (F:145-155, V:360-383)
# ----------------------------------------------------------------------------

def test_default_bounds_match_enumeration():
    b, s, skv, w = 2, 9, 7, 3
    fs, ls, en = R.default_bounds(b, s, skv, w)
    for row in range(b * s):
        bb, i = divmod(row, s)
        legal_full = [bb * skv + j for j in range(skv) if j <= i]
        legal_local = [bb * skv + j for j in range(skv) if j <= i and j >= max(i - w + 1, 0)]
        assert list(range(fs[row], en[row])) == legal_full
        assert list(range(ls[row], en[row])) == legal_local


def test_varlen_metadata_single_sequence_equals_default():
    md = R.varlen_metadata([0, 37], [0, 37], 5)
    fs, ls, en = R.default_bounds(1, 37, 37, 5)
    np.testing.assert_array_equal(md["full_starts"], fs)
    np.testing.assert_array_equal(md["local_starts"], ls)
    np.testing.assert_array_equal(md["causal_ends"], en)
    np.testing.assert_array_equal(md["q_positions"], np.arange(37))
    np.testing.assert_array_equal(md["q_segment_ids"], np.zeros(37))


def test_varlen_metadata_is_shifted_per_sequence():
    cu = [0, 5, 5, 12, 30]
    md = R.varlen_metadata(cu, cu, 4)
    for sidx in range(len(cu) - 1):
        a, b = cu[sidx], cu[sidx + 1]
        fs, ls, en = R.default_bounds(1, b - a, b - a, 4)
        np.testing.assert_array_equal(md["full_starts"][a:b], fs + a)
        np.testing.assert_array_equal(md["local_starts"][a:b], ls + a)
        np.testing.assert_array_equal(md["causal_ends"][a:b], en + a)
        assert (md["q_segment_ids"][a:b] == sidx).all()
        np.testing.assert_array_equal(md["kv_positions"][a:b], np.arange(b - a))
    for k in md:
        assert md[k].dtype == np.int32


# ----------------------------------------------------------------------------
# attention (V:103-249)
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("b,s,hq,hkv,w,p,d", [
    (1, 13, 2, 1, 4, 0.4, 16),
    (2, 9, 4, 2, 3, 0.5, 8),
    (1, 11, 3, 3, 1, 0.3, 8),
    (1, 6, 5, 1, 20, 0.5, 8),
])
def test_attention_matches_float64_brute_force(b, s, hq, hkv, w, p, d):
    q, k, v = _rand_qkv(b * 100 + s, b, s, hq, hkv, d)
    m = _mask(s, (b, s), p)
    o, lse = _routed(q, k, v, m, w)
    ob, lseb = A.brute_force_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                       m.numpy(), w)
    np.testing.assert_allclose(o.numpy(), ob, atol=2e-5, rtol=1e-5)
    np.testing.assert_allclose(lse.numpy(), lseb, atol=2e-5, rtol=1e-5)


def test_attention_varlen_matches_brute_force():
    cu = [0, 4, 5, 13]
    q, k, v = _rand_qkv(7, 1, 13, 4, 2, 8)
    m = _mask(7, (1, 13), 0.5)
    md = R.varlen_metadata(cu, cu, 3)
    o, lse = _routed(q, k, v, m, 3, metadata=md)
    ob, lseb = A.brute_force_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                       m.numpy(), 3, cu_seqlens=cu)
    np.testing.assert_allclose(o.numpy(), ob, atol=2e-5, rtol=1e-5)
    np.testing.assert_allclose(lse.numpy(), lseb, atol=2e-5, rtol=1e-5)


def _sdpa_causal(q, k, v, scale=None):
    """Library routine: causal attention with GQA expanded by repeat_interleave."""
    g = q.shape[2] // k.shape[2]
    qt = q.float().permute(0, 2, 1, 3)
    kt = k.float().repeat_interleave(g, dim=2).permute(0, 2, 1, 3)
    vt = v.float().repeat_interleave(g, dim=2).permute(0, 2, 1, 3)
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=True, scale=scale)
    s = (qt @ kt.transpose(-1, -2)) * (scale if scale is not None else q.shape[-1] ** -0.5)
    s = s.masked_fill(torch.ones(s.shape[-2:], dtype=torch.bool).triu(1), float("-inf"))
    return o.permute(0, 2, 1, 3), torch.logsumexp(s, -1).permute(0, 2, 1) * math.log2(math.e)


def test_all_full_equals_sdpa_causal():
    q, k, v = _rand_qkv(11, 2, 70, 8, 2)
    o, lse = _routed(q, k, v, torch.ones(2, 70, dtype=torch.bool), 16)
    o_ref, lse_ref = _sdpa_causal(q, k, v)
    torch.testing.assert_close(o, o_ref, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(lse, lse_ref, atol=1e-5, rtol=1e-5)


def test_all_full_custom_scale_equals_sdpa_causal():
    q, k, v = _rand_qkv(12, 1, 40, 4, 4)
    o, lse = _routed(q, k, v, torch.ones(1, 40, dtype=torch.bool), 8, sm_scale=0.05)
    o_ref, lse_ref = _sdpa_causal(q, k, v, scale=0.05)
    torch.testing.assert_close(o, o_ref, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(lse, lse_ref, atol=1e-5, rtol=1e-5)


def test_local_with_large_window_equals_causal():
    q, k, v = _rand_qkv(13, 1, 50, 4, 1)
    o_l, lse_l = _routed(q, k, v, torch.zeros(1, 50, dtype=torch.bool), 50)
    o_f, lse_f = _routed(q, k, v, torch.ones(1, 50, dtype=torch.bool), 1)
    torch.testing.assert_close(o_l, o_f, atol=0, rtol=0)
    torch.testing.assert_close(lse_l, lse_f, atol=0, rtol=0)


def test_window_one_returns_own_value_row():
    q, k, v = _rand_qkv(14, 1, 20, 4, 2)
    o, lse = _routed(q, k, v, torch.zeros(1, 20, dtype=torch.bool), 1)
    g = 2
    vv = v.float().repeat_interleave(g, dim=2)
    kk = k.float().repeat_interleave(g, dim=2)
    torch.testing.assert_close(o, vv, atol=1e-6, rtol=0)
    own = (q.float() * kk).sum(-1) * 128 ** -0.5 * math.log2(math.e)
    torch.testing.assert_close(lse, own, atol=1e-5, rtol=1e-5)


def test_sliding_window_by_slicing():
    """Local rows computed by slicing K/V to the window, a different formulation."""
    q, k, v = _rand_qkv(15, 1, 40, 2, 1)
    w = 6
    o, lse = _routed(q, k, v, torch.zeros(1, 40, dtype=torch.bool), w)
    for i in range(40):
        j0 = max(0, i - w + 1)
        for h in range(2):
            s = (k[0, j0:i + 1, 0].float() @ q[0, i, h].float()) * 128 ** -0.5
            p = torch.softmax(s, 0)
            torch.testing.assert_close(o[0, i, h], p @ v[0, j0:i + 1, 0].float(), atol=1e-5,
                                       rtol=1e-5)
            torch.testing.assert_close(lse[0, i, h], torch.logsumexp(s, 0) * math.log2(math.e),
                                       atol=1e-5, rtol=1e-5)


def test_routed_is_rowwise_select_of_branches():
    q, k, v = _rand_qkv(16, 1, 100, 4, 2)
    m = _mask(16, (1, 100), 0.3)
    o, lse = _routed(q, k, v, m, 10)
    o_f, lse_f = _routed(q, k, v, torch.ones(1, 100, dtype=torch.bool), 10)
    o_l, lse_l = _routed(q, k, v, torch.zeros(1, 100, dtype=torch.bool), 10)
    sel = m[0][:, None, None]
    torch.testing.assert_close(o[0], torch.where(sel, o_f[0], o_l[0]), atol=0, rtol=0)
    torch.testing.assert_close(lse[0], torch.where(m[0][:, None], lse_f[0], lse_l[0]),
                               atol=0, rtol=0)


def test_packed_equals_per_sequence():
    cu = [0, 30, 31, 80]
    q, k, v = _rand_qkv(17, 1, 80, 4, 2)
    m = _mask(17, (1, 80), 0.3)
    md = R.varlen_metadata(cu, cu, 8)
    o, lse = _routed(q, k, v, m, 8, metadata=md)
    for a, b in zip(cu[:-1], cu[1:]):
        o_s, lse_s = _routed(q[:, a:b], k[:, a:b], v[:, a:b], m[:, a:b], 8)
        torch.testing.assert_close(o[:, a:b], o_s, atol=1e-6, rtol=1e-6)
        torch.testing.assert_close(lse[:, a:b], lse_s, atol=1e-6, rtol=1e-6)


def test_batch_rows_are_independent():
    q, k, v = _rand_qkv(18, 3, 33, 4, 4)
    m = _mask(18, (3, 33), 0.5)
    o, lse = _routed(q, k, v, m, 5)
    for b in range(3):
        o_b, lse_b = _routed(q[b:b + 1], k[b:b + 1], v[b:b + 1], m[b:b + 1], 5)
        torch.testing.assert_close(o[b:b + 1], o_b, atol=1e-6, rtol=1e-6)
        torch.testing.assert_close(lse[b:b + 1], lse_b, atol=1e-6, rtol=1e-6)


def test_empty_row_is_nan_like_the_reference():
    """A row whose metadata range is empty gives 0/0 = NaN and LSE -inf (V:236-241)."""
    q, k, v = _rand_qkv(19, 1, 4, 1, 1)
    md = R.varlen_metadata([0, 4], [0, 4], 2)
    md["causal_ends"][2] = md["full_starts"][2]
    o, lse = _routed(q, k, v, torch.ones(1, 4, dtype=torch.bool), 2, metadata=md)
    assert torch.isnan(o[0, 2]).all()
    assert lse[0, 2, 0] == float("-inf")


def test_empty_rows_are_nan_in_any_chunk():
    """Rows with no legal key are NaN / -inf whether or not other rows of the
    oracle's chunk have keys: with 10 keys and W = 3, local rows from 12 on
    see none (their start passes the last key), and with chunk = 4 the chunks
    [12, 16) and [16, 20) hold only such rows."""
    q, k, v = _rand_qkv(23, 1, 20, 2, 1, skv=10)
    full, local = R.compact(np.zeros((1, 20), dtype=bool))
    o, lse = oracle.routed_attention(q, k, v, full, local, window_size=3, chunk=4)
    assert torch.isnan(o[0, 12:]).all() and torch.isneginf(lse[0, 12:]).all()
    assert torch.isfinite(o[0, :12]).all() and torch.isfinite(lse[0, :12]).all()
    # the same rows inside mixed chunks agree
    o8, lse8 = oracle.routed_attention(q, k, v, full, local, window_size=3, chunk=8)
    assert torch.equal(torch.isnan(o8), torch.isnan(o))


def test_routed_flops_equals_pair_count():
    m = _mask(20, (2, 77), 0.3)
    full, local = R.compact(m.numpy())
    w = 9
    pairs = 0
    for row in range(2 * 77):
        i = row % 77
        if m.reshape(-1)[row]:
            pairs += i + 1
        else:
            pairs += min(i + 1, w)
    assert A.routed_flops(full, local, 2, 77, 77, 8, 128, w) == 4 * 128 * 8 * pairs


# ----------------------------------------------------------------------------
# planted mistakes: each mutated oracle must fail at least one pin above
# ----------------------------------------------------------------------------

def _pins_pass():
    try:
        test_attention_matches_float64_brute_force(1, 13, 2, 1, 4, 0.4, 16)
        test_attention_matches_float64_brute_force(2, 9, 4, 2, 3, 0.5, 8)
        test_window_one_returns_own_value_row()
        test_all_full_equals_sdpa_causal()
    except AssertionError:
        return False
    return True


_ORIG_BOUNDS = R.default_bounds


def _mut_window_off_by_one(batch, seq_q, seq_kv, window):
    fs, ls, en = _ORIG_BOUNDS(batch, seq_q, seq_kv, window)
    return fs, np.maximum(ls - 1, fs), en


def _mut_causal_off_by_one(batch, seq_q, seq_kv, window):
    fs, ls, en = _ORIG_BOUNDS(batch, seq_q, seq_kv, window)
    en = np.maximum(en - 1, fs + 1)
    return fs, np.minimum(ls, en - 1), en


def test_planted_mistakes_are_caught(monkeypatch):
    assert _pins_pass()
    for mut in (_mut_window_off_by_one, _mut_causal_off_by_one):
        monkeypatch.setattr(A, "default_bounds", mut)
        assert not _pins_pass(), mut.__name__
        monkeypatch.setattr(A, "default_bounds", _ORIG_BOUNDS)
    # LSE without the log2(e) factor
    monkeypatch.setattr(A, "LOG2E", 1.0)
    assert not _pins_pass()
    monkeypatch.setattr(A, "LOG2E", oracle.LOG2E)
    # GQA head mapping h % Hkv instead of h // G: flip the grouping in the oracle
    real_bmm = torch.bmm

    def swapped_bmm(a, b):
        if a.dim() == 3 and a.shape[0] == 2 and b.shape[0] == 2:
            b = b.flip(0)
        return real_bmm(a, b)

    monkeypatch.setattr(A.torch, "bmm", swapped_bmm)
    assert not _pins_pass()
    monkeypatch.setattr(A.torch, "bmm", real_bmm)
    assert _pins_pass()


# ----------------------------------------------------------------------------
# split key ranges: shard bounds and the log2-LSE merge
# ----------------------------------------------------------------------------

def test_shard_bounds_whole_chunk_is_the_default_rule():
    s, w = 300, 37
    fs, ls, e = R.shard_bounds(np.arange(s), 0, s, w)
    dfs, dls, de = R.default_bounds(1, s, s, w)
    assert np.array_equal(fs, dfs) and np.array_equal(ls, dls) and np.array_equal(e, de)


def test_shard_bounds_partition_every_row():
    s, w = 500, 64
    gen = np.random.default_rng(0)
    pos = np.sort(gen.choice(s, size=120, replace=False))
    cuts = [0, 1, 63, 200, 201, 377, s]
    gfs, gls, ge = R.shard_bounds(pos, 0, s, w)
    for starts_g, which in ((gfs, 0), (gls, 1)):
        covered = np.zeros(len(pos), dtype=np.int64)
        for c0, c1 in zip(cuts[:-1], cuts[1:]):
            b = R.shard_bounds(pos, c0, c1, w)
            st, en = b[which], b[2]
            assert np.all(st <= en) and np.all(en <= c1 - c0)
            lo, hi = st + c0, en + c0
            nonempty = hi > lo
            assert np.all(lo[nonempty] >= np.maximum(starts_g, c0)[nonempty])
            assert np.all(hi[nonempty] <= np.minimum(ge, c1)[nonempty])
            covered += hi - lo
        assert np.array_equal(covered, ge - starts_g)


def _attend_keys(q, k, v, keys):
    """float64 attention of each row over an explicit key list (LSE in log2)."""
    n, d = q.shape
    out = np.full((n, d), np.nan)
    lse = np.full(n, -np.inf)
    for i in range(n):
        ks = keys[i]
        if len(ks) == 0:
            continue
        sc = np.array([np.dot(q[i], k[j]) for j in ks]) / math.sqrt(d)
        mx = sc.max()
        wts = np.exp(sc - mx)
        out[i] = (wts[:, None] * v[ks]).sum(0) / wts.sum()
        lse[i] = (mx + math.log(wts.sum())) * oracle.LOG2E
    return out, lse


def test_merge_of_disjoint_key_sets_equals_union():
    gen = np.random.default_rng(3)
    n, nk, d = 30, 50, 16
    q, k, v = gen.normal(size=(n, d)), gen.normal(size=(nk, d)), gen.normal(size=(nk, d))
    rows = [sorted(gen.choice(nk, size=gen.integers(0, 20), replace=False)) for _ in range(n)]
    rows[0] = []                                     # a row with no key at all
    cuts = [0, 10, 11, 35, nk]
    parts = []
    for c0, c1 in zip(cuts[:-1], cuts[1:]):
        parts.append(_attend_keys(q, k, v, [[j for j in r if c0 <= j < c1] for r in rows]))
    o_m, l_m = oracle.merge_partials([p[0] for p in parts], [p[1] for p in parts])
    o_u, l_u = _attend_keys(q, k, v, rows)
    o_m, l_m = o_m.numpy(), l_m.numpy()
    assert np.isnan(o_m[0]).all() and np.isneginf(l_m[0])
    assert np.allclose(o_m, o_u, atol=1e-12, equal_nan=True)   # empty rows: NaN in both
    assert np.allclose(l_m, l_u, atol=1e-12)                   # and -inf in both
    # a natural-log merge (a plausible slip) is caught by the same check
    lt = [torch.as_tensor(p[1]) for p in parts]
    live = np.isfinite(l_u)
    m = torch.stack(lt).amax(0)[live]
    wrong = sum(torch.exp(l[live] - m) for l in lt)
    assert not np.allclose((m + torch.log2(wrong)).numpy(), l_u[live], atol=1e-6)


# ----------------------------------------------------------------------------
# decode: the prefill rule for the last row
# ----------------------------------------------------------------------------

def test_decode_is_the_last_prefill_row():
    gen = torch.Generator().manual_seed(21)
    b, cache_len, hq, hkv, d = 4, 40, 4, 2, 16
    q = torch.randn(b, hq, d, generator=gen)
    k = torch.randn(b, cache_len, hkv, d, generator=gen)
    v = torch.randn(b, cache_len, hkv, d, generator=gen)
    lens = [1, 17, 40, 33]
    for w in (1, 8, 100):
        for full in ([True, False, True, False], [False, True, False, True]):
            o, lse = A.decode_attention(q, k, v, lens, full, window_size=w)
            for i, n in enumerate(lens):
                qs = torch.randn(1, n, hq, d, generator=gen)
                qs[0, n - 1] = q[i]
                mask = np.zeros(n, dtype=bool)
                mask[n - 1] = full[i]
                f, l = R.compact(mask)
                o_p, lse_p = A.routed_attention(qs, k[i:i + 1, :n], v[i:i + 1, :n], f, l,
                                                window_size=w, rows=[n - 1])
                assert torch.allclose(o[i], o_p[0, n - 1], atol=1e-5), (w, i)
                assert torch.allclose(lse[i], lse_p[0, n - 1], atol=1e-5), (w, i)
    # a length beyond the cache is clamped; zero keys give NaN / -inf
    o, lse = A.decode_attention(q, k, v, [0, 99, 1, 1], [True] * 4, window_size=4)
    assert torch.isnan(o[0]).all() and torch.isneginf(lse[0]).all()
    o2, lse2 = A.decode_attention(q, k, v, [0, cache_len, 1, 1], [True] * 4, window_size=4)
    assert torch.equal(o[1], o2[1]) and torch.equal(lse[1], lse2[1])


# ----------------------------------------------------------------------------
# backward: the derivative of the forward restatement
# ----------------------------------------------------------------------------

def _loss_grad_fd(q, k, v, dout, mask, window, cu=None, h=1e-6):
    """Central differences of L = sum(O * dO), O from the float64 brute force."""
    q, k, v, dout = (np.array(x.numpy() if torch.is_tensor(x) else x, dtype=np.float64)
                     for x in (q, k, v, dout))

    def loss():
        o, _ = A.brute_force_attention(q, k, v, mask, window, cu_seqlens=cu)
        return float(np.nansum(o * dout))

    grads = []
    for x in (q, k, v):
        gx = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            i = it.multi_index
            old = x[i]
            x[i] = old + h
            lp = loss()
            x[i] = old - h
            lm = loss()
            x[i] = old
            gx[i] = (lp - lm) / (2 * h)
        grads.append(gx)
    return grads


@pytest.mark.parametrize("b,s,hq,hkv,w,p,d,cu", [
    (1, 7, 4, 2, 3, 0.5, 4, None),
    (2, 5, 2, 1, 2, 0.4, 4, None),
    (1, 8, 2, 2, 2, 0.5, 4, [0, 3, 8]),
])
def test_backward_matches_finite_differences_of_brute_force(b, s, hq, hkv, w, p, d, cu):
    gen = torch.Generator().manual_seed(b * 31 + s)
    q, k, v, do = (torch.randn(b, s, n, d, generator=gen, dtype=torch.float64)
                   for n in (hq, hkv, hkv, hq))
    m = _mask(s + 5, (b, s), p)
    full, local = R.compact(m.numpy())
    md = None if cu is None else R.varlen_metadata(cu, cu, w)
    dq, dk, dv = A.routed_attention_backward(q, k, v, do, full, local, window_size=w,
                                             metadata=md, dtype=torch.float64)
    gq, gk, gv = _loss_grad_fd(q, k, v, do, m.numpy(), w, cu)
    np.testing.assert_allclose(dq.numpy(), gq, atol=1e-7, rtol=1e-6)
    np.testing.assert_allclose(dk.numpy(), gk, atol=1e-7, rtol=1e-6)
    np.testing.assert_allclose(dv.numpy(), gv, atol=1e-7, rtol=1e-6)


@pytest.mark.parametrize("b,s,hq,hkv,w,p,meta", [
    (1, 300, 8, 2, 64, 0.3, False),
    (2, 130, 4, 4, 200, 0.5, False),
    (1, 257, 5, 1, 17, 0.25, True),
])
def test_backward_matches_autograd_of_the_forward(b, s, hq, hkv, w, p, meta):
    gen = torch.Generator().manual_seed(s)
    q, k, v, do = (torch.randn(b, s, n, 32, generator=gen) for n in (hq, hkv, hkv, hq))
    m = _mask(s, (b, s), p)
    full, local = R.compact(m.numpy())
    md = R.varlen_metadata([0, 100, 101, s], [0, 100, 101, s], w) if meta else None
    qa, ka, va = (x.clone().requires_grad_(True) for x in (q, k, v))
    o, _ = A.routed_attention(qa, ka, va, full, local, window_size=w, metadata=md, chunk=64)
    (o * do).sum().backward()
    dq, dk, dv = A.routed_attention_backward(q, k, v, do, full, local, window_size=w,
                                             metadata=md, chunk=96)
    for got, ref in ((dq, qa.grad), (dk, ka.grad), (dv, va.grad)):
        torch.testing.assert_close(got, ref, atol=2e-5, rtol=1e-4)


def test_backward_sum_invariants():
    """sum_j dk_j = 0 (softmax is shift invariant in the keys) and
    sum_j dv_j = sum over the group's rows of dO (each row of P sums to 1)."""
    gen = torch.Generator().manual_seed(3)
    b, s, hq, hkv = 2, 200, 8, 2
    q, k, v, do = (torch.randn(b, s, n, 16, generator=gen) for n in (hq, hkv, hkv, hq))
    full, local = R.compact(_mask(4, (b, s), 0.3).numpy())
    _, dk, dv = A.routed_attention_backward(q, k, v, do, full, local, window_size=32)
    for bb in range(b):
        assert dk[bb].sum(0).abs().max() < 1e-4
        ref = do[bb].reshape(s, hkv, hq // hkv, 16).sum((0, 2))
        torch.testing.assert_close(dv[bb].sum(0), ref, atol=1e-3, rtol=1e-5)


def test_backward_planted_mistakes_are_caught(monkeypatch):
    def pins():
        try:
            test_backward_matches_finite_differences_of_brute_force(1, 7, 4, 2, 3, 0.5, 4, None)
            test_backward_sum_invariants()
        except AssertionError:
            return False
        return True

    assert pins()
    real = A._score_grad
    monkeypatch.setattr(A, "_score_grad", lambda p, dp, delta=None: p * dp)   # Delta dropped
    assert not pins()
    monkeypatch.setattr(A, "_score_grad",
                        lambda p, dp, delta=None: -real(p, dp, delta))        # sign flipped
    assert not pins()
    monkeypatch.setattr(A, "_score_grad", real)
    # GQA head mapping flipped in every product
    real_bmm = torch.bmm

    def swapped_bmm(a, b):
        if a.dim() == 3 and a.shape[0] == 2 and b.shape[0] == 2:
            b = b.flip(0)
        return real_bmm(a, b)

    monkeypatch.setattr(A.torch, "bmm", swapped_bmm)
    assert not pins()
    monkeypatch.setattr(A.torch, "bmm", real_bmm)
    assert pins()


def _few_key_case():
    """Two packed rows of one sequence (cu_seqlens [0, 2], Hq = Hkv = 1,
    window 2, every row local), drawn as the GPU property sweep draws its
    seed-0 case: row 0 sees one key, row 1 two."""
    from switchattentionkernels_amd import workloads
    gen = torch.Generator().manual_seed(0)
    q, k, v = workloads.make_qkv(gen, 1, 2, 2, 1, 1, 128)
    mask = torch.rand((1, 2), generator=gen) < 0.0
    do = torch.randn(q.shape, generator=gen).to(torch.bfloat16)
    full, local = R.compact(mask.numpy())
    return q, k, v, do, full, local, R.varlen_metadata([0, 2], [0, 2], 2)


def _delta_bound_excess(dq, dq_exact, out_used, out_exact, do, terms, rel=1e-2):
    """max over rows of ||dq_r - dq_exact_r|| minus its allowance: the
    Delta-convention shift (``delta_shift_bound``, with 10 % slack for the
    rounding of the other terms) plus rel * ||dq_exact_r|| plus a floor of
    rel times the rms row norm.  <= 0 passes."""
    s = 128 ** -0.5
    dev = (dq.double() - dq_exact.double()).reshape(-1, dq.shape[-2], 128).norm(dim=-1)
    ref = dq_exact.double().reshape(-1, dq.shape[-2], 128).norm(dim=-1)
    allow = (1.1 * A.delta_shift_bound(out_used, out_exact, do, terms["pk"], s)
             + rel * ref + rel * float(ref.pow(2).mean().sqrt()))
    return float((dev - allow).max())


def test_delta_convention_shift_is_the_bound(monkeypatch):
    """The FlashAttention-2 Delta (dO . out with out the bf16 forward output)
    moves dq of a two-key row by 1.45e-2 relative L2 -- above a plain 1e-2 bar
    -- and by exactly scale * |dO . (out - O)| * ||P k|| per row; a dropped or
    doubled Delta lands far outside that bound."""
    q, k, v, do, full, local, md = _few_key_case()
    o, _ = A.routed_attention(q, k, v, full, local, metadata=md)
    ob = o.to(torch.bfloat16)
    terms = {}
    ex = A.routed_attention_backward(q, k, v, do, full, local, metadata=md, delta_terms=terms)
    conv = A.routed_attention_backward(q, k, v, do, full, local, metadata=md, out=ob)
    rel = float((conv[0] - ex[0]).norm() / ex[0].norm())
    assert rel > 1e-2                                  # the plain bar fails here
    shift = A.delta_shift_bound(ob, o, do, terms["pk"], 128 ** -0.5)
    dev = (conv[0] - ex[0]).double().reshape(-1, 1, 128).norm(dim=-1)
    torch.testing.assert_close(dev, shift, rtol=1e-3, atol=1e-5)   # the shift is exact
    assert _delta_bound_excess(conv[0], ex[0], ob, o, do, terms) <= 0
    # The exact O as out gives the exact gradient.
    same = A.routed_attention_backward(q, k, v, do, full, local, metadata=md, out=o)
    torch.testing.assert_close(same[0], ex[0], atol=1e-6, rtol=1e-5)
    real = A._score_grad
    for planted in (lambda p, dp, delta=None: p * dp,                            # dropped
                    lambda p, dp, delta=None: real(p, dp, 2 * delta)):           # doubled
        monkeypatch.setattr(A, "_score_grad", planted)
        bad = A.routed_attention_backward(q, k, v, do, full, local, metadata=md, out=ob)
        assert _delta_bound_excess(bad[0], ex[0], ob, o, do, terms) > 0
        monkeypatch.setattr(A, "_score_grad", real)
