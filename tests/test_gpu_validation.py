"""Validation parity on device tensors: every precondition of the reference's
wrapper fires with the reference's exception type and message, in the
reference's order, before any kernel runs.

* ``_validate_qkv``            V:251-269 (the Hq=32/Hkv=8 pin of V:266-267 is
  relaxed to divisibility, so its branch has no counterpart here);
* ``build_switch_query_indices`` V:313-320;
* metadata checks              V:360-383 (run before the index lists, V:375-386);
* index lists                  V:271-302, V:390-393.

Also: lists built and consumed under ``torch.inference_mode()`` (whose tensors
carry no version counter) give the same result as eager calls, and an in-place
edit made there is still caught by the full device scan.
"""

import re

import pytest
import torch

from switchattentionkernels_amd import (
    build_switch_attention_metadata,
    build_switch_query_indices,
    build_switch_query_indices_from_logits,
    switch_gqa_prefill_backward,
    switch_gqa_prefill_forward,
    workloads,
)

pytestmark = pytest.mark.gpu
DEV = "cuda"

M_DTYPE = "Switch Attention prefill requires BF16 Q/K/V"                   # V:252-253
M_DEVICE = "Q/K/V must be tensors on a supported accelerator device"     # V:254-255
M_CONTIG = "Q/K/V must be contiguous"                                     # V:256-257
M_RANK = "Q/K/V must use [B,S,H,D] layout"                                # V:258-259
M_KV = "K and V must have identical shapes"                               # V:260-261
M_BATCH = "Q and KV batch sizes must match"                               # V:262-263
M_DIM = "the first kernel is specialized for head_dim=128"                # V:264-265
M_HEADS = "query heads must be divisible by KV heads"                     # V:268-269
M_MASK = "full_mask must be a device-resident bool tensor with shape [S] or [1,S]"  # V:318-320
M_META = "invalid Switch Attention position metadata"                     # V:383
M_IDX_DEV = "query indices must be on a supported accelerator device"    # V:281-282
M_RANGE = "query index is outside [0, sequence_length)"                  # V:299-300


def _t(*shape, dtype=torch.bfloat16, device=DEV):
    return torch.zeros(*shape, dtype=dtype, device=device)


def _lists(s):
    idx = torch.arange(s, dtype=torch.int32, device=DEV)
    return idx[::2].contiguous(), idx[1::2].contiguous()


def _expect(exc, msg, q, k, v, s=8, **kw):
    f, l = _lists(s)
    with pytest.raises(exc, match="^" + re.escape(msg) + "$"):
        switch_gqa_prefill_forward(q, k, v, f, l, window_size=4, **kw)


def test_validate_qkv_each_branch():
    s = 8
    q, k, v = _t(1, s, 4, 128), _t(1, s, 2, 128), _t(1, s, 2, 128)
    # V:252-253 dtype, for each of Q, K and V
    _expect(TypeError, M_DTYPE, q.float(), k, v)
    _expect(TypeError, M_DTYPE, q, k.half(), v)
    _expect(TypeError, M_DTYPE, q, k, v.float())
    # V:254-255 device, for each of Q, K and V
    _expect(ValueError, M_DEVICE, q.cpu(), k, v)
    _expect(ValueError, M_DEVICE, q, k.cpu(), v)
    _expect(ValueError, M_DEVICE, q, k, v.cpu())
    # V:256-257 contiguity: transposed views
    _expect(ValueError, M_CONTIG, _t(1, 4, s, 128).transpose(1, 2), k, v)
    _expect(ValueError, M_CONTIG, q, _t(1, 2, s, 128).transpose(1, 2), v)
    _expect(ValueError, M_CONTIG, q, k, _t(1, s, 2, 256)[..., ::2])
    # V:258-259 rank
    _expect(ValueError, M_RANK, _t(s, 4, 128), k, v)
    _expect(ValueError, M_RANK, q, _t(s, 2, 128), _t(s, 2, 128))
    _expect(ValueError, M_RANK, _t(1, 1, s, 4, 128), k, v)
    # V:260-261 K and V shapes
    _expect(ValueError, M_KV, q, k, _t(1, s + 1, 2, 128))
    _expect(ValueError, M_KV, q, k, _t(1, s, 1, 128))
    # V:262-263 batch sizes
    _expect(ValueError, M_BATCH, _t(2, s, 4, 128), k, v)
    # V:264-265 head_dim, on Q and on K/V
    _expect(ValueError, M_DIM, _t(1, s, 4, 64), k, v)
    _expect(ValueError, M_DIM, q, _t(1, s, 2, 64), _t(1, s, 2, 64))
    # V:268-269 head divisibility
    _expect(ValueError, M_HEADS, _t(1, s, 6, 128), _t(1, s, 4, 128), _t(1, s, 4, 128))
    _expect(ValueError, M_HEADS, _t(1, s, 3, 128), k, v)


def test_validate_qkv_order_when_errors_coexist():
    """The first failing check of V:251-269 wins."""
    s = 8
    k, v = _t(1, s, 2, 128), _t(1, s, 2, 128)
    nc_cpu_f32 = torch.zeros(1, 4, s, 128).transpose(1, 2)          # wrong dtype, device, layout
    _expect(TypeError, M_DTYPE, nc_cpu_f32, k, v)                     # dtype before device
    _expect(ValueError, M_DEVICE, nc_cpu_f32.bfloat16(), k, v)        # device before contiguity
    nc_3d = _t(4, s, 128).transpose(0, 1)                             # non-contiguous and 3-D
    _expect(ValueError, M_CONTIG, nc_3d, k, v)                        # contiguity before rank
    _expect(ValueError, M_RANK, _t(s, 4, 128), k, _t(1, s + 1, 2, 128))   # rank before K/V shape
    _expect(ValueError, M_KV, _t(2, s, 4, 128), k, _t(1, s + 1, 2, 128))  # K/V shape before batch
    _expect(ValueError, M_BATCH, _t(2, s, 4, 64), k, v)               # batch before head_dim
    _expect(ValueError, M_DIM, _t(1, s, 3, 64), k, v)                 # head_dim before heads


def test_qkv_checked_before_window_metadata_and_lists():
    s = 8
    q, k, v = _t(1, s, 4, 128), _t(1, s, 2, 128), _t(1, s, 2, 128)
    bad_f = torch.tensor([0, 99], dtype=torch.int32, device=DEV)
    bad_l = torch.tensor([1], dtype=torch.int32)                      # on the CPU
    md = build_switch_attention_metadata(s, s, device=DEV, window_size=4)
    bad_md = md.__class__(**{**md.__dict__, "causal_ends": md.causal_ends.cpu()})
    with pytest.raises(TypeError, match=re.escape(M_DTYPE)):
        switch_gqa_prefill_forward(q.float(), k, v, bad_f, bad_l, window_size=0, metadata=bad_md)
    with pytest.raises(ValueError, match=re.escape("window_size must be positive")):
        switch_gqa_prefill_forward(q, k, v, bad_f, bad_l, window_size=0, metadata=bad_md)
    # metadata (V:375-383) before the index lists (V:384-389)
    with pytest.raises(ValueError, match=re.escape(M_META)):
        switch_gqa_prefill_forward(q, k, v, bad_f, bad_l, window_size=4, metadata=bad_md)
    # the full list's values (V:299-300) before the local list's device (V:281-282)
    with pytest.raises(ValueError, match=re.escape(M_RANGE)):
        switch_gqa_prefill_forward(q, k, v, bad_f, bad_l, window_size=4, metadata=md)
    f, _ = _lists(s)
    with pytest.raises(ValueError, match=re.escape(M_IDX_DEV)):
        switch_gqa_prefill_forward(q, k, v, f, bad_l, window_size=4, metadata=md)


def test_metadata_field_checks():
    """Each field of V:360-374, each condition of V:376-382."""
    s = 16
    q, k, v = _t(1, s, 4, 128), _t(1, s, 2, 128), _t(1, s, 2, 128)
    f, l = _lists(s)
    md = build_switch_attention_metadata(s, s, device=DEV, window_size=4)
    fields = ("q_positions", "kv_positions", "q_segment_ids", "kv_segment_ids", "full_starts",
              "local_starts", "causal_ends")
    for name in fields:
        t = getattr(md, name)
        variants = {
            "cpu": t.cpu(),
            "int64": t.long(),
            "2-D": t.reshape(1, -1),
            "short": t[:-1],
            "long": torch.cat([t, t[:1]]),
            "strided": torch.stack([t, t], dim=1)[:, 0],
        }
        assert not variants["strided"].is_contiguous()
        for tag, bad in variants.items():
            bmd = md.__class__(**{**md.__dict__, name: bad})
            with pytest.raises(ValueError, match="^" + re.escape(M_META) + "$"):
                switch_gqa_prefill_forward(q, k, v, f, l, metadata=bmd)
            print(f"metadata {name} {tag}: rejected", flush=True)
    # the good metadata runs
    o, lse = switch_gqa_prefill_forward(q, k, v, f, l, metadata=md)
    torch.cuda.synchronize()
    assert o.shape == q.shape and lse.shape == q.shape[:3]


def test_mask_checks():
    """V:313-320.  A [B, S] mask with B > 1 is an extension here (flattened
    positions); the reference rejects it with ValueError (V:314-315)."""
    for bad in (torch.zeros(1, 2, 8, dtype=torch.bool, device=DEV),     # 3-D
                torch.zeros(2, 2, 2, dtype=torch.bool, device=DEV),
                torch.zeros((), dtype=torch.bool, device=DEV),          # 0-D
                torch.zeros(8, dtype=torch.int32, device=DEV),          # not bool
                torch.zeros(8, dtype=torch.uint8, device=DEV),
                torch.zeros(1, 8, dtype=torch.float32, device=DEV),
                torch.zeros(8, dtype=torch.bool)):                      # on the CPU
        with pytest.raises(TypeError, match="^" + re.escape(M_MASK) + "$"):
            build_switch_query_indices(bad)
    m = torch.tensor([True, False, True, True], device=DEV)
    for shaped in (m, m[None]):
        f, l = build_switch_query_indices(shaped)
        assert f.tolist() == [0, 2, 3] and l.tolist() == [1]
        assert f.dtype == torch.int32 and l.dtype == torch.int32


def test_inference_mode_lists_and_forward():
    """Lists built under inference_mode are inference tensors with no version
    counter: they are validated in full on every call, and the results equal
    the eager calls bit for bit."""
    gen = torch.Generator().manual_seed(11)
    q, k, v = (t.to(DEV) for t in workloads.make_qkv(gen, 1, 300, 300, 8, 2, 128, 1.0))
    mask = (torch.rand(300, generator=gen) < 0.3).to(DEV)
    logits = torch.randn(300, generator=gen).to(DEV)
    f0, l0 = build_switch_query_indices(mask)
    o0, lse0 = switch_gqa_prefill_forward(q, k, v, f0, l0, window_size=32)
    fl0, ll0 = build_switch_query_indices_from_logits(logits, 0.25)
    with torch.inference_mode():
        f1, l1 = build_switch_query_indices(mask)
        assert f1.is_inference()
        o1, lse1 = switch_gqa_prefill_forward(q, k, v, f1, l1, window_size=32)
        fl1, ll1 = build_switch_query_indices_from_logits(logits, 0.25)
        # an in-place edit under inference_mode is caught by the full scan
        f2, l2 = build_switch_query_indices(mask)
        f2[0], f2[1] = f2[1].clone(), f2[0].clone()
        with pytest.raises(ValueError, match=re.escape("query indices must be strictly increasing")):
            switch_gqa_prefill_forward(q, k, v, f2, l2, window_size=32)
    torch.cuda.synchronize()
    assert torch.equal(f0, f1) and torch.equal(l0, l1)
    assert torch.equal(fl0, fl1) and torch.equal(ll0, ll1)
    assert torch.equal(o0, o1) and torch.equal(lse0, lse1)
    # eager-built lists used inside inference_mode keep their tag and work
    with torch.inference_mode():
        o3, lse3 = switch_gqa_prefill_forward(q, k, v, f0, l0, window_size=32)
        dout = torch.ones_like(q)
        g_inf = switch_gqa_prefill_backward(q, k, v, o1, lse1, dout, f1, l1, window_size=32)
    g_eag = switch_gqa_prefill_backward(q, k, v, o0, lse0, torch.ones_like(q), f0, l0,
                                        window_size=32)
    torch.cuda.synchronize()
    assert torch.equal(o0, o3) and torch.equal(lse0, lse3)
    for a, b in zip(g_inf, g_eag):
        assert torch.equal(a, b)
