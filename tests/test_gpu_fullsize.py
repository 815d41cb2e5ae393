"""Full-size checks at the two largest configurations (#4 packed varlen Hq64,
#5 S=64k Hq40), and a full-size backward check on dK / dV.

* Every routed row is written (V:243-249, V:339-343, V:392-393): O and LSE are
  pre-filled with NaN and passed through the C ABI; every row sees at least its
  own key, so a NaN left behind is a row the kernel never stored.
* Each row depends only on its own route: the routed result equals the
  row-wise select of an all-full and an all-local run (V:134-137) to
  rounding (within 2e-3 on O and 1e-5 on LSE, at most 1 % of the rows
  differing at all): the 256-row kernel takes the exact running max over a
  work item's first two tiles and checks the exponentials of later ones, so
  a row's rounding can depend on the rows that share its work item.
* dK / dV of the late keys (j >= S - 256) against the oracle.  Only the rows of
  the last 256 positions can see those keys (causal, and every window is wider
  than 256), so the oracle restricted to those rows gives those keys' dK / dV
  exactly.  Unlike the sum identities, this fails for a dK that drops a branch,
  a row block or a head.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle
from oracle import routing as R
from switchattentionkernels_amd import (
    build_switch_attention_metadata,
    build_switch_query_indices,
    switch_gqa_prefill_backward,
    switch_gqa_prefill_forward,
    workloads,
)
from switchattentionkernels_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL_L2, REL_MAX = 1e-2, 3e-2


def _inputs(name, seed, **kw):
    wl = workloads.build(name, seed=seed, **kw)
    q, k, v = (wl[x].to(DEV) for x in ("q", "k", "v"))
    md = None
    if wl["cu_seqlens"] is not None:
        t = int(q.shape[1])
        md = build_switch_attention_metadata(t, t, device=DEV, window_size=wl["window"],
                                             cu_seqlens=wl["cu_seqlens"])
    return wl, q, k, v, md


def _abi_forward(q, k, v, full, local, md, window, out, lse):
    """swattn_prefill_fwd straight through the C ABI into caller buffers."""
    b, s, hq, _ = q.shape
    skv, hkv = k.shape[1], k.shape[2]
    L = _lib.lib()
    ws_bytes = L.swattn_prefill_workspace_bytes(b, skv, hkv, 128)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    bounds = ((md.full_starts.data_ptr(), md.local_starts.data_ptr(), md.causal_ends.data_ptr())
              if md is not None else (None, None, None))
    st = L.swattn_prefill_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), full.data_ptr(),
                              full.numel(), local.data_ptr(), local.numel(), *bounds,
                              out.data_ptr(), lse.data_ptr(), b, s, skv, hq, hkv, 128, window,
                              ctypes.c_float(128 ** -0.5 * oracle.LOG2E), ws.data_ptr(),
                              ws_bytes, _lib.stream_handle(q.device))
    assert st == 0, _lib.lib().swattn_last_error()
    torch.cuda.synchronize()


@pytest.mark.parametrize("name,seed", [("varlen", 12), ("s64k", 13)])
def test_every_row_written_canary(name, seed):
    wl, q, k, v, md = _inputs(name, seed)
    print(f"canary {name}: T={q.shape[1]} Hq={q.shape[2]}", flush=True)
    full, local = build_switch_query_indices(wl["mask"].to(DEV))
    assert full.numel() > 0 and local.numel() > 0
    out = torch.full_like(q, float("nan"))
    lse = torch.full(q.shape[:3], float("nan"), device=DEV)
    _abi_forward(q, k, v, full, local, md, wl["window"], out, lse)
    assert not torch.isnan(out).any().item(), "a row of O was never written"
    assert not torch.isnan(lse).any().item(), "a row of LSE was never written"
    assert torch.isfinite(lse).all().item()


@pytest.mark.parametrize("name,seed", [("varlen", 14), ("s64k", 15)])
def test_routed_equals_rowwise_select(name, seed):
    wl, q, k, v, md = _inputs(name, seed)
    m = wl["mask"].to(DEV)
    print(f"row select {name}: T={q.shape[1]} full={int(m.sum())}", flush=True)
    outs = []
    for mask in (m, torch.ones_like(m), torch.zeros_like(m)):
        f, l = build_switch_query_indices(mask)
        outs.append(switch_gqa_prefill_forward(q, k, v, f, l, metadata=md,
                                               window_size=wl["window"]))
    torch.cuda.synchronize()
    (o, lse), (o_f, lse_f), (o_l, lse_l) = outs
    do = (o.float() - torch.where(m[..., None, None], o_f, o_l).float()).abs()
    dl = (lse - torch.where(m[..., None], lse_f, lse_l)).abs()
    rows = int(((do.amax(dim=(-1, -2)) > 0) | (dl.amax(dim=-1) > 0)).sum())
    print(f"row select {name}: rows differing {rows}, max |dO| {float(do.max()):.3e}, "
          f"max |dLSE| {float(dl.max()):.3e}", flush=True)
    assert float(do.max()) <= 2e-3 and float(dl.max()) <= 1e-5
    assert rows <= m.numel() // 100


def _grad_close(got, ref, tag):
    got, ref = got.float().cpu(), ref.float()
    assert torch.isfinite(got).all(), f"{tag}: non-finite gradient"
    err = got - ref
    l2 = float(err.norm() / ref.norm().clamp_min(1e-20))
    mx = float(err.abs().max() / ref.abs().max().clamp_min(1e-20))
    print(f"[grad] {tag}: rel_l2 {l2:.2e} rel_max {mx:.2e}", flush=True)
    assert l2 <= REL_L2 and mx <= REL_MAX, f"{tag}: rel_l2 {l2:.3e} rel_max {mx:.3e}"


@pytest.mark.parametrize("name,seed", [("s16k", 16), ("s64k", 17)])
def test_backward_late_keys_full_size(name, seed):
    wl, q, k, v, _ = _inputs(name, seed)
    s, w = int(q.shape[1]), wl["window"]
    late = 256
    assert w >= late
    gen = torch.Generator().manual_seed(seed)
    do = torch.randn(q.shape, generator=gen).to(torch.bfloat16)
    print(f"backward late keys {name}: S={s}", flush=True)
    full, local = build_switch_query_indices(wl["mask"].to(DEV))
    o, lse = switch_gqa_prefill_forward(q, k, v, full, local, window_size=w)
    dq, dk, dv = switch_gqa_prefill_backward(q, k, v, o, lse, do.to(DEV), full, local,
                                             window_size=w)
    torch.cuda.synchronize()
    f_np, l_np = R.compact(wl["mask"].numpy())
    rows = np.arange(s - late, s)
    rq, rk, rv = oracle.routed_attention_backward(wl["q"], wl["k"], wl["v"], do, f_np, l_np,
                                                  window_size=w, rows=rows, chunk=64)
    _grad_close(dk[0, s - late:], rk[0, s - late:], f"{name} dk of the last {late} keys")
    _grad_close(dv[0, s - late:], rv[0, s - late:], f"{name} dv of the last {late} keys")
    _grad_close(dq[0, s - late:], rq[0, s - late:], f"{name} dq of the last {late} rows")
    # the sampled rows contain both branches
    routed_full = wl["mask"][0, s - late:]
    assert routed_full.any() and (~routed_full).any()
