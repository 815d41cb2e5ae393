"""swattn_decode_fwd_noalloc (library-owned scratch, no workspace argument)
against swattn_decode_fwd (caller workspace), both through the C ABI.

The two share their kernels, so the outputs must be bit-identical.  Two calls
in a row, the second on a smaller problem, show that what the first call left
in the shared scratch does not leak into the second.  A shape whose scratch
need exceeds SWATTN_DECODE_NOALLOC_MAX_BYTES is rejected on the host.
"""

import ctypes
import math

import pytest
import torch

from switchattentionkernels_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"
MAX_BYTES = 16 << 20     # SWATTN_DECODE_NOALLOC_MAX_BYTES in include/swattn.h
LOG2E = 1.4426950408889634


def _problem(seed, batch, cache_len, hq, hkv, p_full):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, hq, 128, generator=gen).to(torch.bfloat16).to(DEV)
    k = torch.randn(batch, cache_len, hkv, 128, generator=gen).to(torch.bfloat16).to(DEV)
    v = torch.randn(batch, cache_len, hkv, 128, generator=gen).to(torch.bfloat16).to(DEV)
    lens = torch.randint(0, cache_len + 1, (batch,), generator=gen, dtype=torch.int32)
    lens[0] = cache_len                        # one sequence fills its cache
    full = (torch.rand(batch, generator=gen) < p_full).to(torch.uint8)
    return q, k, v, lens.to(DEV), full.to(DEV)


def _both(prob, window):
    q, k, v, lens, full = prob
    batch, hq = q.shape[0], q.shape[1]
    cache_len, hkv = k.shape[1], k.shape[2]
    scale = ctypes.c_float(128 ** -0.5 * LOG2E)
    L = _lib.lib()
    need = L.swattn_decode_workspace_bytes(batch, cache_len, hq, hkv)
    assert 0 < need <= MAX_BYTES
    outs = []
    for noalloc in (False, True):
        out = torch.full((batch, hq, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
        lse = torch.full((batch, hq), float("nan"), device=DEV)
        args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), lens.data_ptr(), full.data_ptr(),
                out.data_ptr(), lse.data_ptr(), batch, cache_len, hq, hkv, 128, window, scale)
        with _lib.on_device(q.device):
            if noalloc:
                st = L.swattn_decode_fwd_noalloc(*args, _lib.stream_handle(q.device))
            else:
                ws = torch.empty(need, dtype=torch.uint8, device=DEV)
                st = L.swattn_decode_fwd(*args, ws.data_ptr(), need, _lib.stream_handle(q.device))
        assert st == 0, L.swattn_last_error()
        torch.cuda.synchronize()
        outs.append((out, lse))
    return outs, lens


def _same(a, b):
    """Bit-identical, NaN (empty sequence) included."""
    return torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32),
                       b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32))


def test_noalloc_decode_equals_workspace_decode_twice():
    big = _problem(1, 64, 4096, 32, 8, 0.25)
    small = _problem(2, 5, 700, 40, 8, 0.5)      # smaller, and another group size
    for tag, prob, w in (("B64 L4096 32/8", big, 1024), ("B5 L700 40/8", small, 128)):
        print(f"noalloc decode {tag}", flush=True)
        ((o_ws, l_ws), (o_na, l_na)), lens = _both(prob, w)
        assert _same(o_ws, o_na) and _same(l_ws, l_na), tag
        live = lens.cpu() > 0
        assert torch.isfinite(o_ws.float().cpu()[live]).all()
        assert (torch.isneginf(l_ws.cpu()[~live])).all()


def test_noalloc_decode_rejects_shapes_beyond_its_scratch():
    L = _lib.lib()
    batch, hq, hkv = 4096, 64, 8
    need = L.swattn_decode_workspace_bytes(batch, 64, hq, hkv)
    assert need > MAX_BYTES
    q = torch.zeros(batch, hq, 128, dtype=torch.bfloat16, device=DEV)
    kv = torch.zeros(batch, 64, hkv, 128, dtype=torch.bfloat16, device=DEV)
    lens = torch.zeros(batch, dtype=torch.int32, device=DEV)
    full = torch.zeros(batch, dtype=torch.uint8, device=DEV)
    out = torch.zeros_like(q)
    lse = torch.zeros(batch, hq, device=DEV)
    with _lib.on_device(q.device):
        st = L.swattn_decode_fwd_noalloc(q.data_ptr(), kv.data_ptr(), kv.data_ptr(),
                                         lens.data_ptr(), full.data_ptr(), out.data_ptr(),
                                         lse.data_ptr(), batch, 64, hq, hkv, 128, 64,
                                         ctypes.c_float(0.1), _lib.stream_handle(q.device))
    assert st == -1
    assert b"scratch" in L.swattn_last_error()
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0 and math.isclose(float(lse.abs().sum()), 0.0)
