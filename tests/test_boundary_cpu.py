"""C-ABI and host-logic checks that need no GPU.

The library must load and export every entry point that include/swattn.h
declares, the ctypes signatures must match the header, and argument errors
must be rejected on the host before anything touches a device.
"""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

import oracle
from oracle import routing as R
from switchattentionkernels_amd import _lib, routed_flops, workloads
import switchattentionkernels_amd as sw

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "swattn.h")


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*[\w\s\*]+?\b(swattn_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        args = [a.strip() for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        out[m.group(1)] = len(args)
    return out


def test_library_exports_every_header_symbol():
    funcs = _header_functions()
    assert len(funcs) == 17, funcs
    lib = _lib.lib()
    for name in funcs:
        assert hasattr(lib, name), name
    assert set(funcs) == set(_lib.SIGNATURES)
    for name, nargs in funcs.items():
        assert len(_lib.SIGNATURES[name][1]) == nargs, name


def test_version_and_workspace():
    lib = _lib.lib()
    assert lib.swattn_version() == (0 << 16) | 2
    assert lib.swattn_compact_workspace_bytes(16384) == 0
    assert lib.swattn_compact_workspace_bytes(16385) == 2 * 4
    assert lib.swattn_compact_workspace_bytes(65536) == 4 * 4
    # V^T tiles: Hkv x ceil(B*Skv / 64) x 16 KiB
    assert lib.swattn_prefill_workspace_bytes(2, 100, 8, 128) == 8 * 4 * 16384
    assert lib.swattn_prefill_workspace_bytes(1, 100, 8, 64) == 0
    # backward: per KV head and 32-row block 1 KiB of row info (Q and dO are
    # gathered in place, never copied), one 256-byte zero row, 256-key block
    # ranges (256-byte aligned), and, with fewer than 512 (key tile, KV head)
    # pairs, 256 KiB of fp32 dK/dV partials per split workgroup: here 4 key
    # tiles x 8 KV heads = 32 pairs, split min(16, 512 / 32) = 16 ways.
    # dQ: 5 full and 11 local row tiles of 256 rows, x 8 KV heads; estimated
    # key tiles 17 // 2 + 1 = 9 per full and min(17, 256 / 64 + 2) = 6 per
    # local row tile: 8 * (5 * 9 + 11 * 6) = 888, 4 per slot of 256 (one
    # dQ workgroup per CU).  The longest (17) exceeds that, so row tiles are
    # cut into pieces of max(4, 4) = 4 tiles: 5 slots per full and 2 per
    # local row tile, 128 KiB each, after 128 int32 piece counts (512
    # bytes).
    nb = 8 * (-(-(300 * 4) // 32) + -(-(700 * 4) // 32))
    expect = (nb * 1024 + 256 + 256 + 32 * 16 * 256 * 1024 + 512
              + 8 * (5 * 5 + 11 * 2) * 128 * 1024)
    assert lib.swattn_prefill_bwd_workspace_bytes(1, 1000, 32, 8, 128, 256, 300, 700) == expect
    # config #3 (p_full 0.25 draw): 512 pairs, no dK/dV split; dQ estimate
    # 8 * (63 * 129 + 194 * 18) = 92952, 364 per slot: the longest (257) is
    # under that, no pieces
    nb = 8 * (-(-(4028 * 4) // 32) + -(-(12356 * 4) // 32))
    expect_big = nb * 1024 + 256 + 2 * 64 * 2 * 4     # 64 key tiles x 8 KV heads = 512 pairs
    assert (lib.swattn_prefill_bwd_workspace_bytes(1, 64 * 256, 32, 8, 128, 1024, 4028, 12356)
            == expect_big)
    # its KV-head share (Hq4/Hkv1): 64 pairs split 8 ways; dQ estimate 11619,
    # pieces of 46 tiles per slot: full row tiles get ceil(257 / 46) = 6
    # slots, local ones (18 tiles) one, which writes no partial, so only full
    # slots are kept
    nb = -(-(4028 * 4) // 32) + -(-(12356 * 4) // 32)
    expect_kvh1 = (nb * 1024 + 256 + 2 * 64 * 2 * 4 + 64 * 8 * 256 * 1024 + 1280
                   + 63 * 6 * 128 * 1024)
    assert (lib.swattn_prefill_bwd_workspace_bytes(1, 16384, 4, 1, 128, 1024, 4028, 12356)
            == expect_kvh1)
    # key-range split of the forward: one GPU's share of config #3 split by KV
    # head (Hq4/Hkv1) takes it (chunks of 64 tiles, 5 slots per full item),
    # config #3 itself does not
    base = lib.swattn_prefill_workspace_bytes(1, 16384, 1, 128)
    big = lib.swattn_prefill_split_workspace_bytes(1, 16384, 16384, 4, 1, 128, 1024, 4028, 12356)
    assert big > base
    assert (lib.swattn_prefill_split_workspace_bytes(1, 16384, 16384, 32, 8, 128, 1024, 4028,
                                                     12356)
            == lib.swattn_prefill_workspace_bytes(1, 16384, 8, 128))
    # config #1 (8 full and 24 local items of 128 rows, 2 KV heads): estimate
    # 2 * (8 * (16 // 2 + 2) + 24 * (256 / 64 + 2)) = 448 tiles, 0 per slot of
    # 512, so chunks of the minimum 4 tiles; the longest item (17 tiles) spans
    # more than one and a half, and each full item gets ceil(16 / 4) + 1 = 5
    # slots.  After
    # the V^T tiles (2 x 16 tiles x 16 KiB): fp32 O rows (128 x 128) and LSE
    # (128) per slot, one int2 per full item, each part 256-byte aligned.
    slots = 8 * 2 * 5
    expect1 = 2 * 16 * 16384 + slots * 128 * 128 * 4 + slots * 128 * 4 + 256
    assert (lib.swattn_prefill_split_workspace_bytes(1, 1024, 1024, 8, 2, 128, 256, 256, 768)
            == expect1)
    assert lib.swattn_prefill_split_workspace_bytes(1, 1024, 1024, 8, 3, 128, 256, 256, 768) == 0
    assert lib.swattn_prefill_bwd_workspace_bytes(1, 1000, 30, 8, 128, 256, 300, 700) == 0
    assert lib.swattn_prefill_bwd_workspace_bytes(1, 1000, 32, 8, 64, 256, 300, 700) == 0
    assert lib.swattn_prefill_bwd_workspace_bytes(1, 1000, 32, 8, 128, 0, 300, 700) == 0


def test_host_side_argument_errors():
    lib = _lib.lib()
    # head_dim != 128
    st = lib.swattn_prefill_fwd(None, None, None, None, 1, None, 0, None, None, None, None, None,
                                1, 1, 1, 1, 1, 64, 4, ctypes.c_float(1.0), None, 0, None)
    assert st == -1 and b"head_dim" in lib.swattn_last_error()
    # heads_q not a multiple of heads_kv
    st = lib.swattn_prefill_fwd(None, None, None, None, 1, None, 0, None, None, None, None, None,
                                1, 1, 1, 6, 4, 128, 4, ctypes.c_float(1.0), None, 0, None)
    assert st == -1 and b"multiple" in lib.swattn_last_error()
    # partial metadata
    dummy = ctypes.c_void_p(16)
    st = lib.swattn_prefill_fwd(None, None, None, None, 1, None, 0, dummy, None, None, None, None,
                                1, 1, 1, 4, 4, 128, 4, ctypes.c_float(1.0), None, 0, None)
    assert st == -1 and b"metadata" in lib.swattn_last_error()
    # nothing to do is fine without touching the device
    st = lib.swattn_prefill_fwd(None, None, None, None, 0, None, 0, None, None, None, None, None,
                                1, 0, 1, 4, 4, 128, 4, ctypes.c_float(1.0), None, 0, None)
    assert st == 0
    assert lib.swattn_compact(None, -1, None, None, None, 0, None) == -1
    dummy16 = ctypes.c_void_p(16)
    st = lib.swattn_compact_logits(dummy16, 7, 4, ctypes.c_float(0.0), dummy16, dummy16, None, 0,
                                   None)
    assert st == -1 and b"dtype" in lib.swattn_last_error()
    assert lib.swattn_compact_logits(None, 0, 4, ctypes.c_float(0.0), dummy16, dummy16, None, 0,
                                     None) == -1
    assert lib.swattn_check_indices(None, -1, None, 0, 5, None, None) == -1
    assert lib.swattn_build_metadata(None, None, 1, 4, 4, 0, *([None] * 7), None) == -1
    st = lib.swattn_prefill_bwd(*([dummy16] * 6), dummy16, 1, None, 0, None, None, None,
                                *([dummy16] * 3), 1, 1, 1, 4, 4, 128, 4, ctypes.c_float(0.0),
                                None, 0, None)
    assert st == -1 and b"scale_log2" in lib.swattn_last_error()
    st = lib.swattn_prefill_bwd(*([dummy16] * 6), dummy16, 1, None, 0, dummy16, None, None,
                                *([dummy16] * 3), 1, 1, 1, 4, 4, 128, 4, ctypes.c_float(1.0),
                                None, 0, None)
    assert st == -1 and b"metadata" in lib.swattn_last_error()
    st = lib.swattn_prefill_bwd(*([dummy16] * 6), dummy16, 1, None, 0, None, None, None,
                                *([dummy16] * 3), 1, 1, 1, 4, 4, 128, 4, ctypes.c_float(1.0),
                                None, 0, None)
    assert st == -2 and b"workspace" in lib.swattn_last_error()
    assert not hasattr(lib, "swattn_mfma_peak")       # the probe is not part of the ABI
    probe = _lib.probe_lib()
    assert probe.swattn_mfma_peak(0, 1, dummy16, None) == -1
    assert probe.swattn_mfma_peak(1, 1, None, None) == -1


def test_api_rejects_cpu_and_dtype_errors_like_the_reference():
    q = torch.zeros(1, 8, 4, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16)
    idx = torch.arange(8, dtype=torch.int32)
    with pytest.raises(TypeError, match="requires BF16"):
        sw.switch_gqa_prefill_forward(q.float(), k, k, idx, idx[:0])
    with pytest.raises(ValueError, match="supported accelerator device"):
        sw.switch_gqa_prefill_forward(q, k, k, idx, idx[:0])
    with pytest.raises(TypeError, match="device-resident bool tensor"):
        sw.build_switch_query_indices(torch.zeros(8, dtype=torch.bool))
    with pytest.raises(TypeError, match="float32, bfloat16 or float16"):
        sw.build_switch_query_indices_from_logits(torch.zeros(8))
    with pytest.raises(ValueError, match="supported accelerator device"):
        sw.build_switch_attention_metadata(8, 8, device="cpu", window_size=4)


def test_package_flops_equal_oracle_flops():
    gen = torch.Generator().manual_seed(0)
    for b, s, w, p in ((1, 300, 64, 0.3), (2, 129, 7, 0.5), (1, 50, 100, 1.0)):
        m = torch.rand(b, s, generator=gen) < p
        f, l = R.compact(m.numpy())
        got = routed_flops(torch.from_numpy(f), torch.from_numpy(l), batch=b, seq_q=s, seq_kv=s,
                           heads_q=8, head_dim=128, window=w)
        assert got == oracle.routed_flops(f, l, b, s, s, 8, 128, w)


def test_workloads_are_seeded_and_shaped():
    a = workloads.build("cpu", seed=3)
    b = workloads.build("cpu", seed=3)
    assert torch.equal(a["q"], b["q"]) and torch.equal(a["mask"], b["mask"])
    assert a["q"].shape == (1, 1024, 8, 128) and a["k"].shape == (1, 1024, 2, 128)
    gen = torch.Generator().manual_seed(0)
    mk = workloads.markov_mask(gen, 200000, 0.3)
    assert abs(mk.float().mean().item() - 0.3) < 0.02
    runs = (mk[1:] != mk[:-1]).sum().item()
    assert runs < 200000 * 0.05          # clustered: few switches
    rp = workloads.ramp_mask(gen, 200000)
    assert abs(rp.float().mean().item() - 0.15) < 0.01
    assert rp[:20000].float().mean() < rp[-20000:].float().mean()
    vl = workloads.varlen_lengths(torch.Generator().manual_seed(1))
    assert len(vl) == 8 and all(512 <= x <= 8192 for x in vl)


def test_workspace_partials_stay_within_their_stated_bounds():
    """The workspace queries over many shapes (no GPU needed): the backward's
    dK/dV partials stay within 256 MiB and its dQ partials within 192 MiB
    beyond the row-info blocks, and the forward's split workspace exceeds the
    plain one by at most 200 MiB, as include/swattn.h states."""
    from hypothesis import given, settings, strategies as st

    lib = _lib.lib()
    MiB = 1 << 20

    @settings(max_examples=300, deadline=None, derandomize=True, database=None)
    @given(b=st.integers(1, 8), skv=st.integers(1, 1 << 17), hkv=st.integers(1, 16),
           g=st.sampled_from([1, 2, 4, 5, 8]), w=st.integers(1, 1 << 16),
           frac_full=st.floats(0.0, 1.0), frac_rows=st.floats(0.0, 1.0))
    def check(b, skv, hkv, g, w, frac_full, frac_rows):
        hq = hkv * g
        n = int(b * skv * frac_rows)
        nf = int(n * frac_full)
        nl = n - nf
        bwd = lib.swattn_prefill_bwd_workspace_bytes(b, skv, hq, hkv, 128, w, nf, nl)
        assert bwd > 0
        blocks = hkv * (-(-nf * g // 32) + -(-nl * g // 32))
        kv_tiles = -(-(b * skv) // 256)
        q_items = hkv * (-(-nf * g // 256) + -(-nl * g // 256))
        base = blocks * 1024 + 256 + (2 * kv_tiles * 2 * 4 + 255) // 256 * 256
        extra = bwd - base
        assert 0 <= extra <= 256 * MiB + 192 * MiB + (q_items * 4 + 255) // 256 * 256, \
            (b, skv, hq, hkv, w, nf, nl, bwd, base)
        plain = lib.swattn_prefill_workspace_bytes(b, skv, hkv, 128)
        split = lib.swattn_prefill_split_workspace_bytes(b, skv, skv, hq, hkv, 128, w, nf, nl)
        assert plain <= split <= plain + 200 * MiB, (b, skv, hq, hkv, w, nf, nl, split - plain)

    check()
    # a long sequence with few listed rows: chunk slots bounded by lengthening the chunks
    plain = lib.swattn_prefill_workspace_bytes(1, 129435, 4, 128)
    split = lib.swattn_prefill_split_workspace_bytes(1, 129435, 129435, 16, 4, 128, 10682, 2807, 357)
    assert plain < split <= plain + 200 * MiB
