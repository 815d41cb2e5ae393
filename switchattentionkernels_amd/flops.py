"""Algorithmic work of a routed prefill (the benchmark's FLOP count).

``4 * D * Hq`` FLOPs per legal (query row, key) pair: one multiply-add per
element of Q.K^T and of P.V.  Softmax work is not counted.  Legal keys of a
row are ``[start, end)`` with the bounds of F:145-155 (or the position
metadata, V:134-137), so the count is exact for the mask actually used.
"""

from __future__ import annotations

import torch


def routed_flops(full_idx: torch.Tensor, local_idx: torch.Tensor, *, batch: int, seq_q: int,
                 seq_kv: int, heads_q: int, head_dim: int = 128, window: int = 1024,
                 metadata=None) -> int:
    """Exact routed FLOPs for flattened row lists (any device)."""
    def pairs(idx: torch.Tensor, local: bool) -> int:
        idx = idx.reshape(-1).long()
        if idx.numel() == 0:
            return 0
        if metadata is not None:
            st = (metadata.local_starts if local else metadata.full_starts).long()[idx]
            en = metadata.causal_ends.long()[idx]
        else:
            b = idx // seq_q
            i = idx - b * seq_q
            en = b * seq_kv + torch.clamp(i + 1, max=seq_kv)
            st = b * seq_kv + (torch.clamp(i - window + 1, min=0) if local else 0)
        return int(torch.clamp(en - st, min=0).sum().item())

    return 4 * head_dim * heads_q * (pairs(full_idx, False) + pairs(local_idx, True))
