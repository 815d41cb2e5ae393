"""The forward's 256-row kernel (fwd_wide_kernel) forced on shapes the
library would otherwise give to the 128-row kernel, against the oracle and
against the 128-row kernel.

swattn_prefill_fwd picks the 256-row kernel by itself only for large grids
(1024 work items or more), which the config-sized tests cover; here
SWATTN_FWD_KERNEL=wide / narrow forces one kernel or the other, through the
C ABI with the plain workspace (which never takes the key-range split: with
the public API's split workspace, long full rows on these small grids
would run the 128-row kernel whatever the variable says), on the small
shapes of test_gpu_parity (single and partial tiles, W = 1, W >= S,
G = 1 / 5 / 8, B > 1, Skv != Sq), on packed sequences, on score ranges where
the running maximum moves often (the rescale path) or keys keep rising along
the sequence, and on the masked-tile edge cases (windows shorter than a
64-key tile, rows whose window starts inside a tile), and on keys whose
scores jump far above everything before them (past an item's first two
tiles the kernel exponentiates with the running max as it stands and
checks each half-tile's sums; a failed check, or an exponential beyond the
fp32 range, has the half recomputed with the exact max).  Bars as in
test_gpu_parity (O max-abs <= 2e-2, mean-abs <= 2e-3, LSE relative <= 1e-3;
the NaN / -inf pattern of rows with no key must match the oracle's), for
both kernels; between them O must agree within two bf16 ulps plus 1e-2
and LSE to 1e-3, and the 256-row kernel must be deterministic.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle import routing as R
from switchattentionkernels_amd import (build_switch_attention_metadata, build_switch_query_indices,
                                        switch_gqa_prefill_varlen_forward, workloads)

from test_gpu_parity import SMALL, _assert_close, _mask, _oracle, _qkv

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _plain_run(q, k, v, mask, window, metadata=None, sm_scale=None):
    """swattn_prefill_fwd through the C ABI with the plain workspace
    (swattn_prefill_workspace_bytes).  The public API passes the larger
    split workspace, and where the key-range split is planned (long full
    rows on small grids) it runs the 128-row kernel whatever
    SWATTN_FWD_KERNEL says; with the plain workspace the forced kernel
    runs."""
    import ctypes
    from switchattentionkernels_amd import _lib
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    full, local = build_switch_query_indices(mask.to(DEV))
    b, s, hq, _ = q.shape
    skv, hkv = k.shape[1], k.shape[2]
    L = _lib.lib()
    ws_bytes = L.swattn_prefill_workspace_bytes(b, skv, hkv, 128)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=DEV)
    md = metadata
    scale = (128 ** -0.5 if sm_scale is None else sm_scale) * oracle.LOG2E
    st = L.swattn_prefill_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), full.data_ptr(),
                              full.numel(), local.data_ptr(), local.numel(),
                              _lib.ptr(md.full_starts) if md is not None else None,
                              _lib.ptr(md.local_starts) if md is not None else None,
                              _lib.ptr(md.causal_ends) if md is not None else None,
                              out.data_ptr(), lse.data_ptr(), b, s, skv, hq, hkv, 128, window,
                              ctypes.c_float(scale), ws.data_ptr(), ws_bytes, _lib.stream_handle(q.device))
    assert st == 0, L.swattn_last_error()
    torch.cuda.synchronize()
    return out, lse


def _kernels_agree(ow, lw, on, ln, tag):
    """The two kernels' outputs for the same rows: the same NaN / -inf
    pattern, O within two bf16 ulps of the larger magnitude plus 1e-2 (half
    the oracle bar; the rounding of P moves outputs by a share of |V|, not of
    |O|), LSE within 1e-3 relative.  Each kernel is held to the oracle bars
    separately; between two bf16 results the oracle's absolute bar alone
    would be too tight for large outputs (nearly one-hot rows give |O| up
    to about 5, where one ulp is 0.03)."""
    a, b = ow.float().cpu(), on.float().cpu()
    assert torch.equal(torch.isnan(a), torch.isnan(b)), f"{tag}: NaN patterns differ"
    assert torch.equal(torch.isneginf(lw.cpu()), torch.isneginf(ln.cpu())), f"{tag}: -inf LSE patterns differ"
    fin = ~torch.isnan(a)
    d, mag = (a - b).abs()[fin], torch.maximum(a.abs(), b.abs())[fin]
    worst = float((d - mag * 2 ** -6).max()) if d.numel() else 0.0
    la, lb = lw.cpu(), ln.cpu()
    lf = torch.isfinite(la)
    lrel = float(((la - lb).abs()[lf] / la.abs()[lf].clamp(min=1.0)).max()) if lf.any() else 0.0
    print(f"{tag}: O max {float(d.max()) if d.numel() else 0:.3e} (excess over 2 ulps {worst:.3e}), "
          f"LSE rel {lrel:.3e}", flush=True)
    assert worst <= 1e-2, f"{tag}: O differs by more than two bf16 ulps plus 1e-2"
    assert lrel <= 1e-3, f"{tag}: LSE rel {lrel}"


def _both(monkeypatch, q, k, v, m, w, metadata=None, sm_scale=None):
    monkeypatch.setenv("SWATTN_FWD_KERNEL", "wide")
    ow, lw = _plain_run(q, k, v, m, w, metadata=metadata, sm_scale=sm_scale)
    monkeypatch.setenv("SWATTN_FWD_KERNEL", "narrow")
    on, ln = _plain_run(q, k, v, m, w, metadata=metadata, sm_scale=sm_scale)
    monkeypatch.delenv("SWATTN_FWD_KERNEL")
    return ow, lw, on, ln


@pytest.mark.parametrize("b,s,hq,hkv,w,p,skv", SMALL)
def test_wide_small(monkeypatch, b, s, hq, hkv, w, p, skv):
    q, k, v = _qkv(s * 7 + hq, b, s, hq, hkv, skv)
    m = _mask(s, (b, s), p)
    ow, lw, on, ln = _both(monkeypatch, q, k, v, m, w)
    o_ref, lse_ref = _oracle(q, k, v, m, w)
    tag = f"b{b} s{s} {hq}/{hkv} w{w} p{p} skv{skv}"
    _assert_close(ow, lw, o_ref, lse_ref, tag="wide " + tag)
    _assert_close(on, ln, o_ref, lse_ref, tag="narrow " + tag)
    _kernels_agree(ow, lw, on, ln, tag="wide vs narrow " + tag)


@pytest.mark.parametrize("w", [1, 7, 40, 64, 65, 130])
def test_wide_masked_tiles(monkeypatch, w):
    """Windows from one key to just over two tiles: nearly every tile of a
    local item is a masked tile, with the window start inside a half-tile,
    on a tile edge or crossing the row block's keys."""
    q, k, v = _qkv(31 + w, 1, 777, 8, 2)
    m = _mask(31 + w, (1, 777), 0.3)
    ow, lw, on, ln = _both(monkeypatch, q, k, v, m, w)
    o_ref, lse_ref = _oracle(q, k, v, m, w)
    _assert_close(ow, lw, o_ref, lse_ref, tag=f"wide w{w}")
    _assert_close(on, ln, o_ref, lse_ref, tag=f"narrow w{w}")
    _kernels_agree(ow, lw, on, ln, tag=f"wide vs narrow w{w}")


@pytest.mark.parametrize("qk_scale,sm_scale", [(4.0, None), (1.0, 1.0), (0.05, None), (8.0, 1.0)])
def test_wide_peaked_and_flat_softmax(monkeypatch, qk_scale, sm_scale):
    """Nearly one-hot rows (the running maximum moves often, so the rescale
    of O and l runs) and nearly uniform ones."""
    gen = torch.Generator().manual_seed(21)
    q, k, v = workloads.make_qkv(gen, 1, 700, 700, 8, 2, 128)
    q, k = (q.float() * qk_scale).to(torch.bfloat16), (k.float() * qk_scale).to(torch.bfloat16)
    m = _mask(21, (1, 700), 0.4)
    ow, lw, on, ln = _both(monkeypatch, q, k, v, m, 200, sm_scale=sm_scale)
    o_ref, lse_ref = _oracle(q, k, v, m, 200, sm_scale=sm_scale)
    _assert_close(ow, lw, o_ref, lse_ref, tag=f"wide q,k x{qk_scale} sm_scale {sm_scale}")
    _assert_close(on, ln, o_ref, lse_ref, tag=f"narrow x{qk_scale}")
    _kernels_agree(ow, lw, on, ln, tag=f"wide vs narrow x{qk_scale}")


@pytest.mark.parametrize("gamma", [60.0, 400.0])
def test_wide_score_jumps(monkeypatch, gamma):
    """Every query shares a component along a unit vector u, and a few keys
    carry gamma u: their scores jump by about 3 gamma over every key before
    them, in half 0 and half 1 of tiles 1 to 17 (tile 1 is still taken with
    the exact max; later ones are checked).  gamma 60 puts P near 2^23 over
    the running max (the check fails); gamma 400 puts the exponent past 128,
    so the unchecked exponentials are infinite.  Either way the half is
    recomputed and the rows match the oracle; rows that never see a jump
    are untouched by it."""
    gen = torch.Generator().manual_seed(77)
    s = 1200
    q, k, v = workloads.make_qkv(gen, 1, s, s, 8, 2, 128)
    u = torch.randn(128, generator=gen)
    u = u / u.norm()
    qf, kf = q.float() + 3.0 * u, k.float()
    for pos in (100, 150, 200, 300, 333, 700, 1100):
        kf[0, pos] += gamma * u
    q, k = qf.to(torch.bfloat16), kf.to(torch.bfloat16)
    m = _mask(77, (1, s), 0.4)
    ow, lw, on, ln = _both(monkeypatch, q, k, v, m, 500)
    o_ref, lse_ref = _oracle(q, k, v, m, 500)
    _assert_close(ow, lw, o_ref, lse_ref, tag=f"wide score jumps x{gamma}")
    _assert_close(on, ln, o_ref, lse_ref, tag=f"narrow score jumps x{gamma}")
    _kernels_agree(ow, lw, on, ln, tag=f"wide vs narrow score jumps x{gamma}")


@pytest.mark.parametrize("seed", range(12))
def test_wide_random_jumps(monkeypatch, seed):
    """Randomized checks of the recomputation: a random shape (G = 1, 2, 4
    or 8, so rows start in late tiles too), window and routing, keys with
    jumps of random height along a direction the queries share (from a few
    units to past the fp32 range of 2^x, in either half of random tiles),
    negative jumps (exponentials that underflow), and a few query rows with
    outsized norms."""
    rng = np.random.default_rng(1000 + seed)
    hkv = int(rng.choice([1, 2, 4]))
    g = int(rng.choice([1, 2, 4, 8]))
    s = int(rng.integers(300, 1400))
    w = int(rng.choice([40, 130, 300, 1000, 4096]))
    gen = torch.Generator().manual_seed(seed)
    q, k, v = workloads.make_qkv(gen, 1, s, s, hkv * g, hkv, 128)
    u = torch.randn(128, generator=gen)
    u = u / u.norm()
    qf, kf = q.float() + 3.0 * u, k.float()
    for pos in rng.choice(s, size=int(rng.integers(3, 9)), replace=False):
        kf[0, int(pos), int(rng.integers(hkv))] += float(rng.choice([-200.0, 8.0, 25.0, 60.0, 400.0])) * u
    for row in rng.choice(s, size=4, replace=False):
        qf[0, int(row)] *= 20.0
    q, k = qf.to(torch.bfloat16), kf.to(torch.bfloat16)
    m = _mask(seed, (1, s), float(rng.choice([0.0, 0.3, 1.0])))
    ow, lw, on, ln = _both(monkeypatch, q, k, v, m, w)
    o_ref, lse_ref = _oracle(q, k, v, m, w)
    tag = f"wide random jumps seed {seed}: s{s} g{g} hkv{hkv} w{w}"
    _assert_close(ow, lw, o_ref, lse_ref, tag=tag)
    _assert_close(on, ln, o_ref, lse_ref, tag="narrow " + tag)
    _kernels_agree(ow, lw, on, ln, tag=tag + " vs narrow")


def test_wide_rising_scores(monkeypatch):
    """Keys whose scores against every query rise along the sequence (each
    key a growing multiple of one direction shared with the queries), so
    that the running maximum of a full row moves in almost every half-tile,
    by small and by large steps."""
    s, hq, hkv = 900, 8, 2
    gen = torch.Generator().manual_seed(5)
    q, k, v = workloads.make_qkv(gen, 1, s, s, hq, hkv, 128)
    d = torch.randn(128, generator=gen)
    d = d / d.norm()
    ramp = torch.linspace(0.0, 30.0, s).reshape(1, s, 1, 1)
    jumps = (torch.arange(s) % 97 == 0).float().reshape(1, s, 1, 1) * 25.0
    k = (k.float() * 0.3 + (ramp + jumps) * d).to(torch.bfloat16)
    q = (q.float() * 0.3 + 2.0 * d).to(torch.bfloat16)
    m = _mask(5, (1, s), 0.6)
    ow, lw, on, ln = _both(monkeypatch, q, k, v, m, 300)
    o_ref, lse_ref = _oracle(q, k, v, m, 300)
    _assert_close(ow, lw, o_ref, lse_ref, tag="wide rising scores")
    _assert_close(on, ln, o_ref, lse_ref, tag="narrow rising scores")
    _kernels_agree(ow, lw, on, ln, tag="wide vs narrow rising scores")


def test_wide_varlen(monkeypatch):
    """Packed sequences of uneven lengths (some shorter than a tile, one
    longer than the window) through the varlen entry point."""
    cu = [0, 5, 64, 300, 301, 950, 1400]
    t, hq, hkv, w = cu[-1], 16, 4, 256
    gen = torch.Generator().manual_seed(8)
    q, k, v = workloads.make_qkv(gen, 1, t, t, hq, hkv, 128)
    mask = torch.rand((1, t), generator=gen) < 0.4
    meta = build_switch_attention_metadata(t, t, device=DEV, window_size=w, cu_seqlens=cu)
    ow, lw, on, ln = _both(monkeypatch, q, k, v, mask, w, metadata=meta)
    full, local = build_switch_query_indices(mask.to(DEV))
    api_o, api_l = switch_gqa_prefill_varlen_forward(q.to(DEV), k.to(DEV), v.to(DEV), full, local, cu,
                                                     window_size=w)
    md = R.varlen_metadata(cu, cu, w)
    f_o, l_o = R.compact(mask.numpy())
    o_ref, lse_ref = oracle.routed_attention(q, k, v, f_o, l_o, metadata=md)
    _assert_close(api_o, api_l, o_ref, lse_ref, tag="varlen entry point")
    _assert_close(ow, lw, o_ref, lse_ref, tag="wide varlen")
    _assert_close(on, ln, o_ref, lse_ref, tag="narrow varlen")
    _kernels_agree(ow, lw, on, ln, tag="wide vs narrow varlen")


def test_wide_deterministic_and_every_row_written(monkeypatch):
    """Two calls give bit-identical O and LSE, and every routed row is
    written (outputs pre-filled with NaN)."""
    import ctypes
    from switchattentionkernels_amd import _lib
    monkeypatch.setenv("SWATTN_FWD_KERNEL", "wide")
    b, s, hq, hkv, w = 2, 1500, 32, 8, 512
    q, k, v = (x.to(DEV) for x in _qkv(77, b, s, hq, hkv))
    m = _mask(77, (b, s), 0.35).to(DEV)
    full, local = build_switch_query_indices(m)
    L = _lib.lib()
    ws_bytes = L.swattn_prefill_workspace_bytes(b, s, hkv, 128)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    res = []
    for _ in range(2):
        out = torch.full_like(q, float("nan"))
        lse = torch.full(q.shape[:3], float("nan"), device=DEV)
        st = L.swattn_prefill_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), full.data_ptr(), full.numel(),
                                  local.data_ptr(), local.numel(), None, None, None, out.data_ptr(),
                                  lse.data_ptr(), b, s, s, hq, hkv, 128, w,
                                  ctypes.c_float(128 ** -0.5 * oracle.LOG2E), ws.data_ptr(), ws_bytes,
                                  _lib.stream_handle(q.device))
        assert st == 0, L.swattn_last_error()
        torch.cuda.synchronize()
        res.append((out, lse))
    monkeypatch.delenv("SWATTN_FWD_KERNEL")
    (o1, l1), (o2, l2) = res
    assert not torch.isnan(o1).any() and not torch.isnan(l1).any()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    rows = np.arange(0, b * s, 13)
    o_ref, lse_ref = _oracle(q.cpu(), k.cpu(), v.cpu(), m.cpu(), w, rows=rows)
    _assert_close(o1, l1, o_ref, lse_ref, rows=rows, tag="wide b2 s1500 sampled")


@pytest.mark.parametrize("b,s,hq,hkv,w,p", [(2, 2048, 32, 8, 512, 0.1), (1, 4096, 40, 8, 4096, 0.1),
                                            (1, 6144, 32, 8, 1024, 0.25)])
def test_wide_sparse_full_list_mid_grid(monkeypatch, b, s, hq, hkv, w, p):
    """Grids of 520-776 work items with a sparse full list, where a 256-row
    item's rows spread over hundreds of positions (G = 4 and 5) and its key
    range is the union of theirs: both kernels against the oracle on sampled
    rows and against each other on every row."""
    q, k, v = _qkv(s + hq + w, b, s, hq, hkv)
    m = _mask(s + w, (b, s), p)
    ow, lw, on, ln = _both(monkeypatch, q, k, v, m, w)
    tag = f"b{b} s{s} {hq}/{hkv} w{w} p{p}"
    rows = np.arange(0, b * s, 17)
    o_ref, lse_ref = _oracle(q, k, v, m, w, rows=rows)
    _assert_close(ow, lw, o_ref, lse_ref, rows=rows, tag="wide " + tag)
    _assert_close(on, ln, o_ref, lse_ref, rows=rows, tag="narrow " + tag)
    _kernels_agree(ow, lw, on, ln, tag="wide vs narrow " + tag)
