"""The committed golden fixtures agree with the oracle and with the float64
brute force (CPU only).  The GPU side of the same fixtures is in
test_gpu_parity.py::test_golden_fixture."""

import os

import numpy as np
import pytest
import torch

import oracle
from oracle import routing as R

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
NAMES = sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))


def _load(name):
    z = np.load(os.path.join(GOLDEN, name))
    bf = lambda a: torch.from_numpy(a.astype(np.int16)).view(torch.bfloat16)  # noqa: E731
    cu = z["cu_seqlens"].tolist() if "cu_seqlens" in z.files else None
    return z, bf(z["q"]), bf(z["k"]), bf(z["v"]), z["mask"], int(z["window"]), cu


@pytest.mark.parametrize("name", NAMES)
def test_fixture_reproduced_by_oracle(name):
    z, q, k, v, mask, w, cu = _load(name)
    full, local = R.compact(mask)
    assert np.array_equal(full, z["full_idx"]) and np.array_equal(local, z["local_idx"])
    md = None if cu is None else R.varlen_metadata(cu, cu, w)
    out, lse = oracle.routed_attention(q, k, v, full, local, window_size=w, metadata=md)
    np.testing.assert_allclose(out.numpy(), z["out"], atol=1e-6, rtol=1e-6)
    np.testing.assert_allclose(lse.numpy(), z["lse"], atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("name", NAMES)
def test_fixture_matches_brute_force(name):
    z, q, k, v, mask, w, cu = _load(name)
    ob, lb = oracle.brute_force_attention(q.float().numpy(), k.float().numpy(),
                                          v.float().numpy(), mask, w, cu_seqlens=cu)
    np.testing.assert_allclose(z["out"], ob, atol=2e-5, rtol=1e-5)
    np.testing.assert_allclose(z["lse"], lb, atol=2e-5, rtol=1e-5)
