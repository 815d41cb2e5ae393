"""bench.py's per-workload mode on the GPU: one JSON line per named
workload, with the routed FLOP count the oracle gives for the same mask."""

import argparse
import json
import os
import sys

import pytest

import oracle
from oracle import routing as R
from switchattentionkernels_amd import workloads

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_configs_mode(capsys):
    sys.path.insert(0, ROOT)
    import bench

    bench.config_table(argparse.Namespace(configs="cpu,b2", seed=0))
    lines = [json.loads(x) for x in capsys.readouterr().out.strip().splitlines()]
    assert [x["config"] for x in lines] == ["cpu", "b2"]
    for x in lines:
        assert x["fwd_ms"] > 0 and x["bwd_ms"] > 0
        assert 0 < x["fwd_frac_of_peak"] < 1
        wl = workloads.build(x["config"], seed=0)
        f, l = R.compact(wl["mask"].reshape(-1).numpy())
        q, k = wl["q"], wl["k"]
        flops = oracle.routed_flops(f, l, q.shape[0], q.shape[1], k.shape[1], q.shape[2], 128,
                                    wl["window"])
        assert x["routed_gflop"] == round(flops / 1e9, 1)
