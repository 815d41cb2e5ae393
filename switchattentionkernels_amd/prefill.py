"""Public API of the MI355X Switch Attention prefill (drop-in for the reference).

Mirrors ``swiattn_gqa_prefill_varlen.py`` (V) of YushengZhao/SwitchAttentionKernels:

* ``build_switch_query_indices(full_mask)``          (V:306-322)
* ``switch_gqa_prefill_forward(q, k, v, full_query_indices, local_query_indices, *,
  metadata=None, window_size=1024, sm_scale=None, block_m=64, block_k=64,
  num_stages=1, threads=128) -> (output bf16, lse fp32 log2)``  (V:324-446)

Same argument meaning, same exception types and messages, with the reference's
qualified-shape pins relaxed where the kernels are general:

* any ``Hq`` that is a multiple of ``Hkv`` (V:266-267 pinned 32/8);
* ``B > 1``: index lists then hold flattened positions ``b * S + i`` in
  ``[0, B*S)`` -- exactly what ``build_switch_query_indices`` returns for a
  ``[B, S]`` mask -- and every batch row is its own causal sequence
  (V:346-347 and V:314-315 pinned B = 1);
* a documented-but-unchecked precondition is enforced: the two lists must be
  disjoint (V:341-342).

All device work runs in ``libswattn.so`` (C ABI, ``include/swattn.h``) on
torch's current stream; there is no CPU or PyTorch fallback.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from .metadata import SwitchAttentionMetadata, build_switch_attention_metadata

LOG2E = 1.4426950408889634

MSG_RANGE = "query index is outside [0, sequence_length)"          # V:300
MSG_ORDER = "query indices must be strictly increasing"           # V:302
MSG_COVER = "full and local query lists must cover the sequence"  # V:393
MSG_DISJOINT = "full and local query lists must be disjoint"
MSG_META = "invalid Switch Attention position metadata"           # V:383

ERR_FULL_RANGE, ERR_FULL_ORDER, ERR_LOCAL_RANGE, ERR_LOCAL_ORDER, ERR_OVERLAP = 1, 2, 4, 8, 16


def _validate_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """Preconditions of V:251-269 (Hq/Hkv pin relaxed to divisibility)."""
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError("Switch Attention prefill requires BF16 Q/K/V")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("Q/K/V must be tensors on a supported accelerator device")
    if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
        raise ValueError("Q/K/V must be contiguous")
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("Q/K/V must use [B,S,H,D] layout")
    if k.shape != v.shape:
        raise ValueError("K and V must have identical shapes")
    if q.shape[0] != k.shape[0]:
        raise ValueError("Q and KV batch sizes must match")
    if q.shape[3] != 128 or k.shape[3] != 128:
        raise ValueError("the first kernel is specialized for head_dim=128")
    if k.shape[2] == 0 or q.shape[2] % k.shape[2]:
        raise ValueError("query heads must be divisible by KV heads")
    if not (q.device == k.device == v.device):
        raise ValueError("Q/K/V must be on the same device")


def _prepare_indices(indices: torch.Tensor, *, device: torch.device) -> torch.Tensor:
    """Host-side part of V:271-286: shape, device and int32 cast.

    The reference pads to a power-of-two capacity bucket (V:287-298) only to
    bound TileLang JIT specialisations; the AOT kernels here take the exact
    count, so no padding is made.  The range and order checks (V:299-302) run
    on the device in ``_check_lists``.
    """
    if indices.ndim == 1:
        indices = indices.unsqueeze(0)
    if indices.ndim != 2 or indices.shape[0] != 1:
        raise ValueError("the first kernel accepts one batch of query indices")
    if indices.device.type != "cuda":
        raise ValueError("query indices must be on a supported accelerator device")
    if indices.device != device:
        raise ValueError("query indices must be on the same device as Q")
    return indices.to(dtype=torch.int32).contiguous()[0]


def _device_flags(full: torch.Tensor, local: torch.Tensor, seq_len: int) -> int:
    """Run ``swattn_check_indices``; one 4-byte device-to-host read."""
    flags = torch.empty(1, dtype=torch.int32, device=full.device)
    with _lib.on_device(full.device):
        st = _lib.lib().swattn_check_indices(full.data_ptr(), full.numel(), local.data_ptr(),
                                             local.numel(), seq_len, flags.data_ptr(),
                                             _lib.stream_handle(full.device))
    _lib.check(st, "swattn_check_indices")
    return int(flags.item())


def _raise_for(flags: int, which: str) -> None:
    if which == "full":
        if flags & ERR_FULL_RANGE:
            raise ValueError(MSG_RANGE)
        if flags & ERR_FULL_ORDER:
            raise ValueError(MSG_ORDER)
    else:
        if flags & ERR_LOCAL_RANGE:
            raise ValueError(MSG_RANGE)
        if flags & ERR_LOCAL_ORDER:
            raise ValueError(MSG_ORDER)


class _Compaction:
    """Identity of one ``build_switch_query_indices`` result (``n`` positions)."""

    __slots__ = ("n",)

    def __init__(self, n: int):
        self.n = n


def _tag_compacted(full: torch.Tensor, local: torch.Tensor, n: int) -> None:
    """Mark a fresh compaction result.  Both lists are ascending, disjoint and
    cover ``[0, n)`` by construction; torch's version counter (shared by the
    two views of one buffer) shows whether either was modified since.

    Inference tensors (made under ``torch.inference_mode()``) have no version
    counter, so an in-place edit could not be seen: they are left untagged and
    every forward call scans them in full."""
    if full.is_inference():
        return
    token = _Compaction(n)
    full._swattn_compaction = (token, "full", full._version)
    local._swattn_compaction = (token, "local", local._version)


def _is_untouched_compaction(full, local, seq_len: int) -> bool:
    a = getattr(full, "_swattn_compaction", None)
    b = getattr(local, "_swattn_compaction", None)
    return (a is not None and b is not None and a[0] is b[0] and a[0].n == seq_len
            and a[1] == "full" and b[1] == "local"
            and not full.is_inference() and not local.is_inference()
            and full._version == a[2] and local._version == b[2])


def _check_lists(full_query_indices, local_query_indices, seq_len: int, device):
    """V:384-393 in the reference's order, plus disjointness last.

    A pair returned by ``build_switch_query_indices`` for this sequence length
    and not modified since is valid by construction: only the device check
    runs for it, and the device-side scan and its blocking read are skipped.
    """
    if _is_untouched_compaction(full_query_indices, local_query_indices, seq_len):
        if full_query_indices.device != device or local_query_indices.device != device:
            raise ValueError("query indices must be on the same device as Q")
        return full_query_indices, local_query_indices
    full = _prepare_indices(full_query_indices, device=device)
    try:
        local = _prepare_indices(local_query_indices, device=device)
    except ValueError:
        # The reference checks the full list's values before the local list's shape.
        _raise_for(_device_flags(full, full[:0], seq_len), "full")
        raise
    flags = _device_flags(full, local, seq_len)
    _raise_for(flags, "full")
    _raise_for(flags, "local")
    if full.numel() + local.numel() != seq_len:
        raise ValueError(MSG_COVER)
    if flags & ERR_OVERLAP:
        raise ValueError(MSG_DISJOINT)
    return full, local


def _check_metadata(metadata: SwitchAttentionMetadata, q_len: int, kv_len: int, device) -> None:
    """V:360-383."""
    tensors = (metadata.q_positions, metadata.kv_positions, metadata.q_segment_ids,
               metadata.kv_segment_ids, metadata.full_starts, metadata.local_starts,
               metadata.causal_ends)
    expected = (q_len, kv_len, q_len, kv_len, q_len, q_len, q_len)
    for t, n in zip(tensors, expected):
        if (t.device != device or t.dtype != torch.int32 or t.ndim != 1 or t.numel() != n
                or not t.is_contiguous()):
            raise ValueError(MSG_META)


def build_switch_query_indices(full_mask: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Compact a hard route mask into sorted full and local query positions.

    ``True`` routes to full causal attention and ``False`` to sliding-window
    attention (V:306-322).  A ``[1, S]`` or ``[S]`` mask gives positions in
    ``[0, S)``; a ``[B, S]`` mask (an extension: V:314-315 rejects B > 1) gives
    flattened positions ``b * S + i``.  Both lists are ascending int32 device
    tensors, bit-identical to ``arange(n)[mask]`` and ``arange(n)[~mask]``.
    One device-to-host read fetches the split point, as torch's boolean
    indexing does in the reference.
    """
    if full_mask.ndim == 2:
        full_mask = full_mask.reshape(-1)
    if full_mask.ndim != 1 or full_mask.dtype != torch.bool or not full_mask.is_cuda:
        raise TypeError(
            "full_mask must be a device-resident bool tensor with shape [S] or [1,S]"
        )
    n = full_mask.numel()
    if n >= 2 ** 31:
        raise ValueError("full_mask must hold fewer than 2^31 positions")
    dev = full_mask.device
    mask = full_mask.contiguous()
    out = torch.empty(n, dtype=torch.int32, device=dev)
    counts = torch.empty(2, dtype=torch.int32, device=dev)
    L = _lib.lib()
    ws_bytes = int(L.swattn_compact_workspace_bytes(n))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    with _lib.on_device(dev):
        st = L.swattn_compact(mask.data_ptr(), n, out.data_ptr(), counts.data_ptr(),
                              ws.data_ptr(), ws_bytes, _lib.stream_handle(dev))
    _lib.check(st, "swattn_compact")
    nf = int(counts[0].item())
    full, local = out[:nf], out[nf:]
    _tag_compacted(full, local, n)
    return full, local


_LOGIT_DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def build_switch_query_indices_from_logits(
        router_logits: torch.Tensor, threshold: float = 0.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Route and compact in one pass: full attention where ``router_logits >
    threshold``.

    Same result, bit for bit, as ``build_switch_query_indices(router_logits >
    threshold)``, without materialising the mask.  The reference keeps its
    router outside the kernels (README:85, V:4-5); this is the fused step in
    front of ``build_switch_query_indices`` (V:306-322).  ``router_logits`` is
    a device tensor of shape ``[S]``, ``[1, S]`` or ``[B, S]`` (positions then
    flattened to ``b * S + i``) in float32, bfloat16 or float16.  As with
    torch's ``>`` against a Python number, the threshold is first rounded to
    the logits' dtype.
    """
    if router_logits.ndim == 2:
        router_logits = router_logits.reshape(-1)
    if (router_logits.ndim != 1 or router_logits.dtype not in _LOGIT_DTYPES
            or not router_logits.is_cuda):
        raise TypeError("router_logits must be a device-resident float32, bfloat16 or float16 "
                        "tensor with shape [S], [1,S] or [B,S]")
    n = router_logits.numel()
    if n >= 2 ** 31:
        raise ValueError("router_logits must hold fewer than 2^31 positions")
    dev = router_logits.device
    logits = router_logits.contiguous()
    thr = float(torch.tensor(float(threshold), dtype=logits.dtype).item())
    out = torch.empty(n, dtype=torch.int32, device=dev)
    counts = torch.empty(2, dtype=torch.int32, device=dev)
    L = _lib.lib()
    ws_bytes = int(L.swattn_compact_workspace_bytes(n))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    with _lib.on_device(dev):
        st = L.swattn_compact_logits(logits.data_ptr(), _LOGIT_DTYPES[logits.dtype], n, thr,
                                     out.data_ptr(), counts.data_ptr(), ws.data_ptr(), ws_bytes,
                                     _lib.stream_handle(dev))
    _lib.check(st, "swattn_compact_logits")
    nf = int(counts[0].item())
    full, local = out[:nf], out[nf:]
    _tag_compacted(full, local, n)
    return full, local


def switch_gqa_prefill_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    full_query_indices: torch.Tensor,
    local_query_indices: torch.Tensor,
    *,
    metadata: Optional[SwitchAttentionMetadata] = None,
    window_size: int = 1024,
    sm_scale: Optional[float] = None,
    block_m: int = 64,
    block_k: int = 64,
    num_stages: int = 1,
    threads: int = 128,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Run Switch Attention prefill forward.

    Returns BF16 output ``[B, Sq, Hq, 128]`` and FP32 log2-LSE ``[B, Sq, Hq]``.
    The two index lists must be sorted, disjoint, and together cover every
    query position exactly once (V:339-343).  ``metadata`` overrides the
    per-row key bounds (then ``window_size`` is only checked to be positive,
    as in V); without it the bounds follow F:145-155 inside each batch row.
    ``block_m``, ``block_k``, ``num_stages`` and ``threads`` are accepted for
    compatibility; values other than the reference's qualified schedule raise
    ``AssertionError`` as the reference kernel does (V:67-71).
    """
    _validate_qkv(q, k, v)
    if window_size <= 0:
        raise ValueError("window_size must be positive")
    batch, q_len, heads, dim = (int(x) for x in q.shape)
    kv_len, kv_heads = int(k.shape[1]), int(k.shape[2])
    if metadata is not None and batch != 1:
        raise ValueError("position metadata requires batch size 1; pack sequences with cu_seqlens")
    if kv_len == 0 and q_len > 0:
        raise ValueError("K/V must hold at least one position")
    total_q = batch * q_len
    if metadata is not None:
        _check_metadata(metadata, q_len, kv_len, q.device)
    full, local = _check_lists(full_query_indices, local_query_indices, total_q, q.device)

    output = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
    if total_q == 0:
        return output, lse
    assert block_m == 64, "the qualified schedule is BM64"
    assert block_k == 64, "the qualified schedule is BK64"
    assert num_stages == 1, "the qualified schedule uses one stage"
    assert threads == 128, "the qualified schedule uses 128 threads"
    scale = ((1.0 / dim) ** 0.5 if sm_scale is None else float(sm_scale)) * LOG2E
    md = metadata
    L = _lib.lib()
    # The larger workspace that lets the kernel split long full items by key
    # range when they would otherwise set its length (few KV heads).
    ws_bytes = int(L.swattn_prefill_split_workspace_bytes(batch, q_len, kv_len, heads, kv_heads,
                                                          dim, int(window_size), full.numel(),
                                                          local.numel()))
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    with _lib.on_device(q.device):
        st = L.swattn_prefill_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(),
            full.data_ptr(), full.numel(), local.data_ptr(), local.numel(),
            _lib.ptr(md.full_starts) if md is not None else None,
            _lib.ptr(md.local_starts) if md is not None else None,
            _lib.ptr(md.causal_ends) if md is not None else None,
            output.data_ptr(), lse.data_ptr(), batch, q_len, kv_len, heads, kv_heads, dim,
            int(window_size), scale, workspace.data_ptr(), ws_bytes,
            _lib.stream_handle(q.device))
    _lib.check(st, "swattn_prefill_fwd")
    return output, lse


def switch_gqa_prefill_varlen_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    full_query_indices: torch.Tensor,
    local_query_indices: torch.Tensor,
    cu_seqlens,
    *,
    cu_seqlens_kv=None,
    window_size: int = 1024,
    sm_scale: Optional[float] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Packed-sequence prefill: ``q``/``k``/``v`` are ``[1, T, H, 128]`` with
    the sequences concatenated along T at offsets ``cu_seqlens``.  Builds the
    position metadata (``build_switch_attention_metadata``) and calls
    ``switch_gqa_prefill_forward``; attention never crosses a sequence."""
    _validate_qkv(q, k, v)
    md = build_switch_attention_metadata(int(q.shape[1]), int(k.shape[1]), device=q.device,
                                         window_size=window_size, cu_seqlens=cu_seqlens,
                                         cu_seqlens_kv=cu_seqlens_kv)
    return switch_gqa_prefill_forward(q, k, v, full_query_indices, local_query_indices,
                                      metadata=md, window_size=window_size, sm_scale=sm_scale)
