"""Routed decode: one new query token per sequence against its KV cache.

The reference is prefill-only.  This applies its routing rule to the last row
of a sequence (F:145-155): with ``n = cache_lens[b]`` the new token sits at
position ``n - 1`` -- its own K/V already appended -- and attends keys
``[0, n)`` when routed full, else the last ``window_size`` of them.  Output
follows the prefill's conventions: bf16 O and fp32 LSE in the log2
convention (V:15, V:236-241).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

LOG2E = 1.4426950408889634


def switch_gqa_decode_forward(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                              cache_lens: torch.Tensor, full_mask: torch.Tensor, *,
                              window_size: int = 1024,
                              sm_scale: Optional[float] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Routed decode step.

    ``q``: bf16 ``[B, 1, Hq, 128]`` (or ``[B, Hq, 128]``); ``k_cache`` /
    ``v_cache``: bf16 ``[B, L, Hkv, 128]``; ``cache_lens``: int32 ``[B]``
    (valid cache rows, new token included; clamped to ``[0, L]``);
    ``full_mask``: bool ``[B]``, True = full attention over the cache.
    Returns ``(O [B, 1, Hq, 128] bf16, LSE [B, 1, Hq] fp32)``.
    """
    squeeze = q.ndim == 3
    if squeeze:
        q = q.unsqueeze(1)
    for t in (q, k_cache, v_cache):
        if t.dtype != torch.bfloat16:
            raise TypeError("Switch Attention decode requires BF16 Q and KV cache")
        if not t.is_cuda:
            raise ValueError("Q and KV cache must be tensors on a supported accelerator device")
        if not t.is_contiguous():
            raise ValueError("Q and KV cache must be contiguous")
    if q.ndim != 4 or q.shape[1] != 1 or k_cache.ndim != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("q must be [B,1,Hq,128] and the caches [B,L,Hkv,128] of one shape")
    batch, _, heads, dim = (int(x) for x in q.shape)
    _, cache_len, kv_heads, kdim = (int(x) for x in k_cache.shape)
    if dim != 128 or kdim != 128:
        raise ValueError("the decode kernel is specialized for head_dim=128")
    if k_cache.shape[0] != batch:
        raise ValueError("Q and KV cache batch sizes must match")
    if kv_heads == 0 or heads % kv_heads or heads // kv_heads > 8:
        raise ValueError("query heads must be a multiple (at most 8x) of KV heads")
    if cache_len == 0:
        raise ValueError("the KV cache must hold at least one position")
    if window_size <= 0:
        raise ValueError("window_size must be positive")
    dev = q.device
    if (cache_lens.dtype != torch.int32 or cache_lens.shape != (batch,)
            or cache_lens.device != dev):
        raise ValueError("cache_lens must be an int32 [B] tensor on the device of Q")
    if full_mask.dtype != torch.bool or full_mask.shape != (batch,) or full_mask.device != dev:
        raise ValueError("full_mask must be a bool [B] tensor on the device of Q")
    if not (k_cache.device == v_cache.device == dev):
        raise ValueError("Q and KV cache must be on the same device")
    scale = ((1.0 / dim) ** 0.5 if sm_scale is None else float(sm_scale)) * LOG2E
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=dev)
    lens = cache_lens.contiguous()
    full = full_mask.contiguous().view(torch.uint8)
    L = _lib.lib()
    ws_bytes = int(L.swattn_decode_workspace_bytes(batch, cache_len, heads, kv_heads))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    with _lib.on_device(dev):
        st = L.swattn_decode_fwd(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                 lens.data_ptr(), full.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                 batch, cache_len, heads, kv_heads, dim, int(window_size), scale,
                                 ws.data_ptr(), ws_bytes, _lib.stream_handle(dev))
    _lib.check(st, "swattn_decode_fwd")
    if squeeze:
        return out[:, 0], lse[:, 0]
    return out, lse
