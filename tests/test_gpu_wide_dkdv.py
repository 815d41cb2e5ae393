"""The backward's 64-key-per-wave dK/dV kernel (bwd_dkdv_wide_kernel)
against the oracle and against the eight-wave dK/dV kernel.

The 64-key kernel is the default; under 512 (key tile, KV head) pairs it
shares each pair's row blocks out over several workgroups whose fp32
partials the reduce kernel adds, as the eight-wave kernel does.
SWATTN_DKDV_KERNEL=wide names it explicitly on the small shapes below (all
split), =narrow forces the eight-wave kernel.  Both take the same split and
the same dQ kernel, so dq agrees bit for bit.  Their dk and dv differ in
rounding only:
the 64-key kernel takes a pair's full-branch row blocks from the last down
(the eight-wave kernel from the first up), so the fp32 sums run in another
order, and it takes dP - Delta from the matrix cores (the accumulation
starts from Delta, against negated V rows) where the eight-wave kernel
subtracts Delta afterwards.  They agree to rel. L2 2e-3 and 1 % of the
largest element, far inside the oracle bars.

The forced shapes cover single and partial tiles, G = 1 / 5 / 8, B > 1,
Skv != Sq (key tiles past the last row, rows with no key), windows shorter
than a tile (masked blocks), nearly one-hot and nearly uniform rows and
packed sequences with metadata; each dk and dv is held to the oracle at
the bar of test_gpu_backward.
"""

import pytest
import torch

from switchattentionkernels_amd import build_switch_attention_metadata

from test_gpu_backward import _grad_close, _mask, _md_np, _oracle, _qkv, _run

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _forced(monkeypatch, kind, *args, **kw):
    monkeypatch.setenv("SWATTN_DKDV_KERNEL", kind)
    out = _run(*args, **kw)
    monkeypatch.delenv("SWATTN_DKDV_KERNEL")
    return out


def _check(got, ref, tag):
    for g, r, n in zip(got, ref, ("dq", "dk", "dv")):
        _grad_close(g, r, f"{tag} {n}")


@pytest.mark.parametrize("b,s,hq,hkv,w,p,skv", [
    (1, 300, 8, 2, 64, 0.3, None),      # G = 4, ragged length
    (2, 257, 4, 4, 100, 0.5, None),     # G = 1, two batch rows
    (1, 520, 40, 8, 128, 0.25, None),   # G = 5: blocks straddle query positions
    (1, 200, 64, 8, 1, 0.2, None),      # G = 8, window 1
    (1, 1000, 32, 8, 1024, 0.25, None), # window beyond the sequence
    (1, 384, 8, 2, 96, 0.0, None),      # all local
    (1, 384, 8, 2, 96, 1.0, None),      # all full
    (1, 300, 8, 2, 64, 0.4, 180),       # fewer keys than queries
    (2, 200, 8, 2, 50, 0.3, 333),       # more keys than queries: key tiles no row sees
    (3, 512, 8, 2, 100, 0.3, None),     # whole 256-key tiles per sequence
    (3, 164, 8, 1, 2, 0.3, 3),          # late local rows with empty ranges
])
def test_wide_dkdv_matches_oracle(monkeypatch, b, s, hq, hkv, w, p, skv):
    q, k, v, do = _qkv(b * 1000 + s + 5, b, s, hq, hkv, skv)
    m = _mask(s + hq + 2, (b, s), p)
    tag = f"wide dkdv b{b} s{s} {hq}/{hkv} w{w} p{p} skv{skv}"
    got = _forced(monkeypatch, "wide", q, k, v, do, m, w)
    _check(got, _oracle(q, k, v, do, m, w), tag)


@pytest.mark.parametrize("w", [1, 7, 40, 64, 65, 130])
def test_wide_dkdv_masked_blocks(monkeypatch, w):
    """Windows from one key to just over two tiles: most blocks of a key
    tile are masked blocks."""
    q, k, v, do = _qkv(60 + w, 1, 777, 8, 2)
    m = _mask(60 + w, (1, 777), 0.3)
    got = _forced(monkeypatch, "wide", q, k, v, do, m, w)
    _check(got, _oracle(q, k, v, do, m, w), f"wide dkdv w{w}")


@pytest.mark.parametrize("qk_scale", [4.0, 0.05])
def test_wide_dkdv_peaked_and_flat(monkeypatch, qk_scale):
    q, k, v, do = _qkv(31, 1, 600, 8, 2)
    q, k = (q.float() * qk_scale).to(torch.bfloat16), (k.float() * qk_scale).to(torch.bfloat16)
    m = _mask(31, (1, 600), 0.4)
    got = _forced(monkeypatch, "wide", q, k, v, do, m, 150)
    _check(got, _oracle(q, k, v, do, m, 150), f"wide dkdv q,k x{qk_scale}")


def test_wide_dkdv_varlen_metadata(monkeypatch):
    cu = [0, 5, 64, 300, 301, 950, 1400]
    t, hq, hkv, w = cu[-1], 16, 4, 256
    q, k, v, do = _qkv(14, 1, t, hq, hkv)
    m = _mask(14, (1, t), 0.4)
    md = build_switch_attention_metadata(t, t, device=DEV, window_size=w, cu_seqlens=cu)
    got = _forced(monkeypatch, "wide", q, k, v, do, m, w, metadata=md)
    _check(got, _oracle(q, k, v, do, m, w, md_np=_md_np(md)), "wide dkdv varlen")


@pytest.mark.parametrize("b,s,hq,hkv,w,p", [
    (1, 8192, 16, 16, 512, 0.3),     # 32 key tiles x 16 KV heads = 512 pairs: no split
    (2, 4096, 32, 16, 300, 0.5),     # two sequences, 512 pairs
    (2, 4096, 32, 8, 1024, 0.25),    # 256 pairs: split in two
    (1, 16384, 4, 1, 1024, 0.25),    # one KV head, 64 pairs: split in eight
    (1, 1024, 8, 2, 256, 0.25),      # 8 pairs: the largest split
])
def test_wide_dkdv_matches_eight_wave(monkeypatch, b, s, hq, hkv, w, p):
    """The default (64-key) kernel's dk and dv match the eight-wave
    kernel's within the bar above (dq bit for bit), split or not, and reruns
    are bit-identical."""
    q, k, v, do = _qkv(b * 7 + s, b, s, hq, hkv)
    m = _mask(s + 9, (b, s), p)
    wide = _run(q, k, v, do, m, w)
    again = _run(q, k, v, do, m, w)
    narrow = _forced(monkeypatch, "narrow", q, k, v, do, m, w)
    for name, a, c, n in zip(("dq", "dk", "dv"), wide, again, narrow):
        a32, n32 = a.float(), n.float()
        diff = float((a32 - n32).abs().max())
        l2 = float((a32 - n32).norm() / n32.norm().clamp_min(1e-20))
        print(f"[wide dkdv] b{b} s{s} {name}: max |wide - narrow| = {diff:.3e}, rel L2 {l2:.2e}", flush=True)
        assert torch.equal(a, c), f"{name}: reruns differ"
        if name == "dq":
            assert torch.equal(a, n), f"dq: the two runs differ by {diff:.3e}"
        else:
            assert l2 <= 2e-3 and diff <= 1e-2 * float(n32.abs().max()), f"{name}: rel L2 {l2:.2e}, max {diff:.3e}"
