"""Position metadata for Switch Attention prefill.

The reference imports ``SwitchAttentionMetadata`` and
``build_switch_attention_metadata`` from a sibling module ``.metadata``
(V:27) that it does not ship.  Its wrapper calls the builder as
``build_switch_attention_metadata(q_len, kv_len, device=..., window_size=...)``
(V:353-359), checks seven int32 vectors (V:360-383), and the kernel reads
``full_starts``/``local_starts``/``causal_ends`` per query row (V:134-137,
V:186-193): row q may attend key j iff ``start(q) <= j < causal_ends(q)``.

This module provides that interface, built on the GPU by
``swattn_build_metadata``.  For one sequence the bounds equal the fixed-length
kernel's rule (F:145-155).  With ``cu_seqlens`` the rule applies inside each
packed sequence, so attention never crosses a sequence boundary.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib


@dataclass(frozen=True)
class SwitchAttentionMetadata:
    """Per-row key bounds and positions; every field is int32, 1-D, contiguous.

    ``q_positions``/``q_segment_ids``/``full_starts``/``local_starts``/
    ``causal_ends`` have one entry per query row and ``kv_positions``/
    ``kv_segment_ids`` one per key row (lengths checked as in V:374).
    ``*_starts`` and ``causal_ends`` are key-row indices.
    """

    q_positions: torch.Tensor
    kv_positions: torch.Tensor
    q_segment_ids: torch.Tensor
    kv_segment_ids: torch.Tensor
    full_starts: torch.Tensor
    local_starts: torch.Tensor
    causal_ends: torch.Tensor


def _as_cu(cu, total: int, name: str) -> list:
    vals = [int(x) for x in (cu.tolist() if isinstance(cu, torch.Tensor) else cu)]
    if len(vals) < 2 or vals[0] != 0:
        raise ValueError(f"{name} must start at 0 and hold at least one sequence")
    if any(b < a for a, b in zip(vals, vals[1:])):
        raise ValueError(f"{name} must be non-decreasing")
    if vals[-1] != total:
        raise ValueError(f"{name} must end at the packed length {total}")
    return vals


def build_switch_attention_metadata(q_len: int, kv_len: int, *, device, window_size: int,
                                    cu_seqlens=None, cu_seqlens_kv=None) -> SwitchAttentionMetadata:
    """Build position metadata for ``q_len`` query rows and ``kv_len`` key rows.

    Without ``cu_seqlens`` the rows form one sequence.  ``cu_seqlens`` (int
    list or tensor of ``nseq + 1`` offsets) packs several sequences; keys use
    ``cu_seqlens_kv`` when given, else the same offsets.  Inside a sequence,
    query i sees keys ``[ks, ks + min(i + 1, kv_len_seq))`` (full) or
    ``[ks + max(i - W + 1, 0), ...)`` (local), ``ks`` being the sequence's
    first key row.
    """
    q_len, kv_len, window_size = int(q_len), int(kv_len), int(window_size)
    if window_size <= 0:
        raise ValueError("window_size must be positive")
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError("metadata must be built on a supported accelerator device")
    cq = _as_cu([0, q_len] if cu_seqlens is None else cu_seqlens, q_len, "cu_seqlens")
    ck_src = cu_seqlens_kv if cu_seqlens_kv is not None else (
        [0, kv_len] if cu_seqlens is None else cu_seqlens)
    ck = _as_cu(ck_src, kv_len, "cu_seqlens_kv")
    if len(ck) != len(cq):
        raise ValueError("cu_seqlens and cu_seqlens_kv must describe the same number of sequences")
    cq_t = torch.tensor(cq, dtype=torch.int32, device=dev)
    ck_t = torch.tensor(ck, dtype=torch.int32, device=dev)

    def e(n):
        return torch.empty(n, dtype=torch.int32, device=dev)

    md = SwitchAttentionMetadata(e(q_len), e(kv_len), e(q_len), e(kv_len), e(q_len), e(q_len),
                                 e(q_len))
    with _lib.on_device(dev):
        st = _lib.lib().swattn_build_metadata(
            cq_t.data_ptr(), ck_t.data_ptr(), len(cq) - 1, q_len, kv_len, window_size,
            md.q_positions.data_ptr(), md.kv_positions.data_ptr(), md.q_segment_ids.data_ptr(),
            md.kv_segment_ids.data_ptr(), md.full_starts.data_ptr(), md.local_starts.data_ptr(),
            md.causal_ends.data_ptr(), _lib.stream_handle(dev))
    _lib.check(st, "swattn_build_metadata")
    return md
