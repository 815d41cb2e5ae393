"""The backward's 256-row dQ kernel (bwd_dq_wide_kernel, the default) against
the 32-row-wave dQ kernel (SWATTN_DQ_KERNEL=narrow) and the oracle.

Both kernels compute P = 2^(c s - LSE) with the same fp32 operations and
accumulate S and dQ in the same k-step order.  The 256-row kernel starts
its dP accumulation from -Delta (so the matrix cores return dP - Delta)
where the 32-row-wave kernel subtracts Delta afterwards: their dS differ
in rounding only, and so their dq agree to rel. L2 2e-3 and 1 % of the
largest element; dk and dv come from the same kernel either way and agree
bit for bit.  The shapes cover single and partial tiles,
G = 1 / 5 / 8, B > 1, Skv != Sq, rows with no key (dq = 0), windows shorter
than a tile or starting inside one (masked tiles), nearly one-hot and nearly
uniform rows, packed sequences with metadata, and row tiles cut into pieces
(fp32 partials summed by the reduce kernel).  Each dq is also held to the
oracle at the bar of test_gpu_backward.
"""

import numpy as np
import pytest
import torch

from switchattentionkernels_amd import build_switch_attention_metadata

from test_gpu_backward import _grad_close, _mask, _md_np, _oracle, _qkv, _run

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _both(monkeypatch, *args, **kw):
    monkeypatch.setenv("SWATTN_DQ_KERNEL", "narrow")
    narrow = _run(*args, **kw)
    monkeypatch.delenv("SWATTN_DQ_KERNEL")
    wide = _run(*args, **kw)
    return wide, narrow


def _same(wide, narrow, tag):
    for name, a, b in zip(("dq", "dk", "dv"), wide, narrow):
        a32, b32 = a.float(), b.float()
        diff = float((a32 - b32).abs().max()) if a.numel() else 0.0
        l2 = float((a32 - b32).norm() / b32.norm().clamp_min(1e-20)) if a.numel() else 0.0
        print(f"[wide dq] {tag} {name}: max |wide - narrow| = {diff:.3e}, rel L2 {l2:.2e}", flush=True)
        if name == "dq":
            big = float(b32.abs().max()) if b.numel() else 0.0
            assert l2 <= 2e-3 and diff <= 1e-2 * big, f"{tag} dq: rel L2 {l2:.2e}, max {diff:.3e}"
        else:
            assert torch.equal(a, b), f"{tag} {name}: the two runs differ by {diff:.3e}"


@pytest.mark.parametrize("b,s,hq,hkv,w,p,skv", [
    (1, 300, 8, 2, 64, 0.3, None),      # G = 4, ragged length, pieces
    (2, 257, 4, 4, 100, 0.5, None),     # G = 1, two batch rows
    (1, 520, 40, 8, 128, 0.25, None),   # G = 5
    (1, 200, 64, 8, 1, 0.2, None),      # G = 8, window 1
    (1, 1000, 32, 8, 1024, 0.25, None), # window beyond the sequence
    (1, 384, 8, 2, 96, 1.0, None),      # all full
    (2, 300, 8, 2, 64, 0.3, 100),       # fewer keys than queries: rows with no key
    (2, 200, 8, 2, 50, 0.3, 333),       # more keys than queries
    (1, 4096, 4, 1, 256, 0.3, None),    # pieces of 4 tiles
    (1, 2000, 32, 8, 1024, 0.25, None), # no pieces, long full rows
])
def test_wide_dq_matches_narrow_and_oracle(monkeypatch, b, s, hq, hkv, w, p, skv):
    q, k, v, do = _qkv(b * 1000 + s + 3, b, s, hq, hkv, skv)
    m = _mask(s + hq + 1, (b, s), p)
    tag = f"b{b} s{s} {hq}/{hkv} w{w} p{p} skv{skv}"
    wide, narrow = _both(monkeypatch, q, k, v, do, m, w)
    _same(wide, narrow, tag)
    rq, _, _ = _oracle(q, k, v, do, m, w)
    _grad_close(wide[0], rq, tag + " dq")


@pytest.mark.parametrize("w", [1, 7, 40, 64, 65, 130])
def test_wide_dq_masked_tiles(monkeypatch, w):
    """Windows from one key to just over two tiles: nearly every tile of a
    local row tile is masked, with window starts inside a half-tile, on a
    tile edge or crossing the row block's keys."""
    q, k, v, do = _qkv(40 + w, 1, 777, 8, 2)
    m = _mask(40 + w, (1, 777), 0.3)
    wide, narrow = _both(monkeypatch, q, k, v, do, m, w)
    _same(wide, narrow, f"w{w}")
    rq, _, _ = _oracle(q, k, v, do, m, w)
    _grad_close(wide[0], rq, f"w{w} dq")


@pytest.mark.parametrize("qk_scale", [4.0, 0.05])
def test_wide_dq_peaked_and_flat(monkeypatch, qk_scale):
    q, k, v, do = _qkv(29, 1, 600, 8, 2)
    q, k = (q.float() * qk_scale).to(torch.bfloat16), (k.float() * qk_scale).to(torch.bfloat16)
    m = _mask(29, (1, 600), 0.4)
    wide, narrow = _both(monkeypatch, q, k, v, do, m, 150)
    _same(wide, narrow, f"q,k x{qk_scale}")
    rq, _, _ = _oracle(q, k, v, do, m, 150)
    _grad_close(wide[0], rq, f"q,k x{qk_scale} dq")


def test_wide_dq_varlen_metadata(monkeypatch):
    """Packed sequences (one shorter than a tile, one of a single row)
    through caller metadata."""
    cu = [0, 5, 64, 300, 301, 950, 1400]
    t, hq, hkv, w = cu[-1], 16, 4, 256
    q, k, v, do = _qkv(12, 1, t, hq, hkv)
    m = _mask(12, (1, t), 0.4)
    md = build_switch_attention_metadata(t, t, device=DEV, window_size=w, cu_seqlens=cu)
    wide, narrow = _both(monkeypatch, q, k, v, do, m, w, metadata=md)
    _same(wide, narrow, "varlen")
    rq, _, _ = _oracle(q, k, v, do, m, w, md_np=_md_np(md))
    _grad_close(wide[0], rq, "varlen dq")


def test_wide_dq_deterministic_on_a_large_grid():
    """Config #2's shape (B2 S4096 Hq32/Hkv8 W1024): two calls give
    bit-identical dq, and sampled rows match the oracle."""
    q, k, v, do = _qkv(202, 2, 4096, 32, 8)
    m = _mask(202, (2, 4096), 0.25)
    a = _run(q, k, v, do, m, 1024)
    c = _run(q, k, v, do, m, 1024)
    assert torch.equal(a[0], c[0])
    rows = np.unique(np.random.default_rng(5).choice(2 * 4096, 256, replace=False))
    rq, _, _ = _oracle(q, k, v, do, m, 1024, rows=rows)
    _grad_close(a[0], rq, "b2 dq sampled rows", rows=torch.as_tensor(rows))
