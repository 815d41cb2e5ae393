"""Routed prefill over split key ranges: the pieces context parallelism needs.

The reference runs one device over the whole key range.  Its metadata already
separates query from key positions (V:139-141, V:179-182), and it exports the
log2 LSE (V:15, V:236-241).  With those, a query shard can attend one key
chunk at a time and the partial results can be combined exactly:

* ``shard_attention_metadata`` gives the per-row key bounds of query rows at
  global positions against a key chunk ``[kv_start, kv_end)``, in chunk
  coordinates (F:145-155 cut to the chunk);
* ``merge_attention_partials`` combines partial (O, LSE) results over
  disjoint key ranges into the result over their union.

Both run in ``libswattn.so`` (``swattn_shard_bounds``,
``swattn_merge_partials``).
"""

from __future__ import annotations

import ctypes
from typing import Sequence, Tuple

import torch

from . import _lib
from .metadata import SwitchAttentionMetadata


def shard_attention_metadata(q_positions: torch.Tensor, *, kv_start: int, kv_end: int,
                             window_size: int) -> SwitchAttentionMetadata:
    """Metadata for query rows at global positions ``q_positions`` of one causal
    sequence against the keys ``[kv_start, kv_end)`` of that sequence.

    Pass it to ``switch_gqa_prefill_forward`` with ``k``/``v`` holding exactly
    that key chunk.  Row ``r`` may attend global keys ``[0, p]`` (full) or
    ``[p - window_size + 1, p]`` (local), ``p = q_positions[r]``, cut to the
    chunk; a row with no key there gets an empty range, and the forward
    returns O = NaN, LSE = -inf for it, which the merge ignores.
    """
    if q_positions.ndim != 1 or q_positions.dtype != torch.int32 or not q_positions.is_cuda:
        raise TypeError("q_positions must be a device-resident 1-D int32 tensor")
    if not (0 <= kv_start <= kv_end):
        raise ValueError("need 0 <= kv_start <= kv_end")
    if window_size <= 0:
        raise ValueError("window_size must be positive")
    dev = q_positions.device
    pos = q_positions.contiguous()
    n = pos.numel()
    full_starts = torch.empty(n, dtype=torch.int32, device=dev)
    local_starts = torch.empty_like(full_starts)
    causal_ends = torch.empty_like(full_starts)
    with _lib.on_device(dev):
        st = _lib.lib().swattn_shard_bounds(pos.data_ptr(), n, int(kv_start), int(kv_end),
                                            int(window_size), full_starts.data_ptr(),
                                            local_starts.data_ptr(), causal_ends.data_ptr(),
                                            _lib.stream_handle(dev))
    _lib.check(st, "swattn_shard_bounds")
    kv_len = int(kv_end) - int(kv_start)
    return SwitchAttentionMetadata(
        q_positions=pos,
        kv_positions=torch.arange(kv_start, kv_end, dtype=torch.int32, device=dev),
        q_segment_ids=torch.zeros(n, dtype=torch.int32, device=dev),
        kv_segment_ids=torch.zeros(kv_len, dtype=torch.int32, device=dev),
        full_starts=full_starts, local_starts=local_starts, causal_ends=causal_ends)


def merge_attention_partials(outputs: Sequence[torch.Tensor],
                             lses: Sequence[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    """Combine partial results over disjoint key ranges (up to 16 parts).

    ``outputs[i]``: bf16 ``[B, S, Hq, 128]``; ``lses[i]``: fp32 ``[B, S, Hq]``
    in the log2 convention, as ``switch_gqa_prefill_forward`` returns them.
    Returns ``(O, LSE)`` over the union of the key ranges:
    ``LSE = log2(sum_i 2^LSE_i)`` and ``O = sum_i 2^(LSE_i - LSE) O_i``.
    """
    if len(outputs) != len(lses) or not 1 <= len(outputs) <= 16:
        raise ValueError("need 1 to 16 partial (O, LSE) pairs")
    o0, l0 = outputs[0], lses[0]
    for o, l in zip(outputs, lses):
        if o.dtype != torch.bfloat16 or l.dtype != torch.float32:
            raise TypeError("partial outputs must be bf16 and partial LSEs fp32")
        if (o.shape != o0.shape or l.shape != l0.shape or o.shape[:-1] != l.shape
                or o.shape[-1] != 128):
            raise ValueError("partials must share the shapes [B, S, Hq, 128] / [B, S, Hq]")
        if not (o.is_cuda and l.is_cuda and o.device == o0.device and l.device == o0.device):
            raise ValueError("partials must be on one accelerator device")
    outs = [o.contiguous() for o in outputs]
    ls = [l.contiguous() for l in lses]
    out = torch.empty_like(outs[0])
    lse = torch.empty_like(ls[0])
    n = len(outs)
    o_ptrs = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    l_ptrs = (ctypes.c_void_p * n)(*[l.data_ptr() for l in ls])
    dev = out.device
    with _lib.on_device(dev):
        st = _lib.lib().swattn_merge_partials(o_ptrs, l_ptrs, n, out.data_ptr(), lse.data_ptr(),
                                              lse.numel(), 128, _lib.stream_handle(dev))
    _lib.check(st, "swattn_merge_partials")
    return out, lse
