"""Backward pass of the routed GQA prefill, and an autograd-enabled wrapper.

The reference is forward-only (V:14-15, V = ``swiattn_gqa_prefill_varlen.py``);
these compute the derivative of its forward (V:103-249) in
``swattn_prefill_bwd`` (``include/swattn.h``), from the forward's output and
its log2 LSE (V:236-241):

* ``switch_gqa_prefill_backward(q, k, v, output, lse, grad_output,
  full_query_indices, local_query_indices, *, metadata=None, window_size=1024,
  sm_scale=None) -> (dq, dk, dv)``, all bf16 in the shapes of q, k, v;
* ``switch_gqa_prefill(q, k, v, full_query_indices, local_query_indices, *,
  metadata=None, window_size=1024, sm_scale=None) -> (output, lse)``: the
  forward of ``switch_gqa_prefill_forward`` as a ``torch.autograd.Function``
  whose output is differentiable in q, k and v (the LSE output is not);
* ``switch_gqa_prefill_varlen(q, k, v, full_query_indices,
  local_query_indices, cu_seqlens, *, cu_seqlens_kv=None, window_size=1024,
  sm_scale=None)``: the same for packed sequences.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from .metadata import SwitchAttentionMetadata, build_switch_attention_metadata
from .prefill import (LOG2E, MSG_META, _check_lists, _check_metadata, _validate_qkv,
                      switch_gqa_prefill_forward)


def _check_monotone(metadata: SwitchAttentionMetadata, full: torch.Tensor,
                    local: torch.Tensor) -> None:
    """The backward finds the rows that see a key block by binary search, so
    each list's key bounds must be non-decreasing along the list (true for
    every single causal sequence and for packed sequences in order).  A
    start past its row's end is an empty range and counts as the end, as in
    the kernels.  One device-to-host read."""
    ok = torch.ones((), dtype=torch.bool, device=full.device)
    for lst, starts in ((full, metadata.full_starts), (local, metadata.local_starts)):
        if lst.numel() > 1:
            li = lst.long()
            ends = metadata.causal_ends[li]
            for b in (torch.minimum(starts[li], ends), ends):
                ok = ok & (b[1:] >= b[:-1]).all()
    if not bool(ok.item()):
        raise ValueError(MSG_META + ": key bounds must be non-decreasing along each index list "
                         "for the backward pass")


def switch_gqa_prefill_backward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    output: torch.Tensor,
    lse: torch.Tensor,
    grad_output: torch.Tensor,
    full_query_indices: torch.Tensor,
    local_query_indices: torch.Tensor,
    *,
    metadata: Optional[SwitchAttentionMetadata] = None,
    window_size: int = 1024,
    sm_scale: Optional[float] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradients of ``switch_gqa_prefill_forward``'s output with respect to
    q, k and v, given ``grad_output`` (same shape as the output).

    ``output`` and ``lse`` are that forward's results for the same arguments.
    Returns ``(dq, dk, dv)`` in bf16; a query row that sees no key gets
    ``dq = 0`` and a key row that no query sees gets ``dk = dv = 0``.
    """
    _validate_qkv(q, k, v)
    if window_size <= 0:
        raise ValueError("window_size must be positive")
    for name, t, dt in (("output", output, torch.bfloat16), ("grad_output", grad_output,
                                                              torch.bfloat16)):
        if t.shape != q.shape or t.dtype != dt or t.device != q.device or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous BF16 tensor shaped like Q")
    if (lse.shape != q.shape[:3] or lse.dtype != torch.float32 or lse.device != q.device
            or not lse.is_contiguous()):
        raise ValueError("lse must be a contiguous FP32 tensor shaped [B, Sq, Hq]")
    batch, q_len, heads, dim = (int(x) for x in q.shape)
    kv_len, kv_heads = int(k.shape[1]), int(k.shape[2])
    if metadata is not None and batch != 1:
        raise ValueError("position metadata requires batch size 1; pack sequences with cu_seqlens")
    total_q = batch * q_len
    if metadata is not None:
        _check_metadata(metadata, q_len, kv_len, q.device)
    full, local = _check_lists(full_query_indices, local_query_indices, total_q, q.device)
    if metadata is not None:
        _check_monotone(metadata, full, local)
    scale = ((1.0 / dim) ** 0.5 if sm_scale is None else float(sm_scale))
    if not scale > 0:
        raise ValueError("sm_scale must be positive")
    # The lists cover every query position once (checked above), and the
    # kernels write every listed row (0 for a row with no key): no fill.
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    md = metadata
    L = _lib.lib()
    ws_bytes = int(L.swattn_prefill_bwd_workspace_bytes(batch, kv_len, heads, kv_heads, dim,
                                                        int(window_size), full.numel(),
                                                        local.numel()))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    with _lib.on_device(q.device):
        st = L.swattn_prefill_bwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), output.data_ptr(), lse.data_ptr(),
            grad_output.data_ptr(), full.data_ptr(), full.numel(), local.data_ptr(),
            local.numel(),
            _lib.ptr(md.full_starts) if md is not None else None,
            _lib.ptr(md.local_starts) if md is not None else None,
            _lib.ptr(md.causal_ends) if md is not None else None,
            dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), batch, q_len, kv_len, heads, kv_heads,
            dim, int(window_size), scale * LOG2E, workspace.data_ptr(), ws_bytes,
            _lib.stream_handle(q.device))
    _lib.check(st, "swattn_prefill_bwd")
    return dq, dk, dv


class SwitchGQAPrefillFunction(torch.autograd.Function):
    """Routed prefill with a backward: ``apply(q, k, v, full, local, metadata,
    window_size, sm_scale) -> (output, lse)``; lse is not differentiable."""

    @staticmethod
    def forward(ctx, q, k, v, full, local, metadata, window_size, sm_scale):
        out, lse = switch_gqa_prefill_forward(q, k, v, full, local, metadata=metadata,
                                              window_size=window_size, sm_scale=sm_scale)
        ctx.save_for_backward(q, k, v, out, lse, full, local)
        ctx.md = metadata
        ctx.window_size = window_size
        ctx.sm_scale = sm_scale
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, grad_out, grad_lse):
        q, k, v, out, lse, full, local = ctx.saved_tensors
        g = grad_out.to(torch.bfloat16).contiguous()
        dq, dk, dv = switch_gqa_prefill_backward(q, k, v, out, lse, g, full, local,
                                                 metadata=ctx.md,
                                                 window_size=ctx.window_size,
                                                 sm_scale=ctx.sm_scale)
        return dq, dk, dv, None, None, None, None, None


def switch_gqa_prefill(q, k, v, full_query_indices, local_query_indices, *,
                       metadata: Optional[SwitchAttentionMetadata] = None,
                       window_size: int = 1024,
                       sm_scale: Optional[float] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """``switch_gqa_prefill_forward`` with autograd support for q, k, v."""
    return SwitchGQAPrefillFunction.apply(q, k, v, full_query_indices, local_query_indices,
                                          metadata, window_size, sm_scale)


def switch_gqa_prefill_varlen(q, k, v, full_query_indices, local_query_indices, cu_seqlens, *,
                              cu_seqlens_kv=None, window_size: int = 1024,
                              sm_scale: Optional[float] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """``switch_gqa_prefill_varlen_forward`` with autograd support for q, k, v:
    ``q``/``k``/``v`` are ``[1, T, H, 128]`` with the sequences concatenated
    along T at offsets ``cu_seqlens``."""
    _validate_qkv(q, k, v)
    md = build_switch_attention_metadata(int(q.shape[1]), int(k.shape[1]), device=q.device,
                                         window_size=window_size, cu_seqlens=cu_seqlens,
                                         cu_seqlens_kv=cu_seqlens_kv)
    return switch_gqa_prefill(q, k, v, full_query_indices, local_query_indices, metadata=md,
                              window_size=window_size, sm_scale=sm_scale)
