"""Write the golden fixtures under tests/golden/ (run from the repo root).

The reference ships no golden vectors and cannot run here (TileLang + Hopper),
so the expected outputs come from this repository's CPU oracle, which is pinned
separately (float64 brute force, SDPA, closed forms); tests/test_golden_cpu.py
re-derives every fixture with both the oracle and the float64 brute force.

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from oracle import routing as R  # noqa: E402

CASES = [
    # name, batch, seq, hq, hkv, window, p_full, cu_seqlens
    ("single_s96_h4x2_w16", 1, 96, 4, 2, 16, 0.3, None),
    ("varlen_3seq_h5x1_w8", 1, 90, 5, 1, 8, 0.4, [0, 40, 41, 90]),
    ("batch2_s70_h2x2_w5", 2, 70, 2, 2, 5, 0.5, None),
]


def make(name, batch, seq, hq, hkv, window, p, cu, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, seq, hq, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(batch, seq, hkv, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(batch, seq, hkv, 128, generator=g).to(torch.bfloat16)
    mask = torch.rand(batch, seq, generator=g) < p
    full, local = R.compact(mask.numpy())
    md = None if cu is None else R.varlen_metadata(cu, cu, window)
    out, lse = oracle.routed_attention(q, k, v, full, local, window_size=window, metadata=md)
    arrays = dict(
        q=q.view(torch.int16).numpy(), k=k.view(torch.int16).numpy(),
        v=v.view(torch.int16).numpy(), mask=mask.numpy(), window=np.int64(window),
        full_idx=full, local_idx=local, out=out.numpy(), lse=lse.numpy())
    if cu is not None:
        arrays["cu_seqlens"] = np.asarray(cu, dtype=np.int32)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)


if __name__ == "__main__":
    for i, case in enumerate(CASES):
        make(*case, seed=100 + i)
        print("wrote", case[0])
