"""Benchmark: routed GQA prefill on one MI355X.

Metric: routed-attention TFLOP/s and ms per prefill at
S=16k Hq32/Hkv8, plus the fraction of bf16 MFMA peak.

Workload (the config the metric is quoted on): B=1, S=16384, Hq=32, Hkv=8,
d=128, window 1024, Bernoulli(p_full=0.25) routing, bf16 N(0,1) inputs drawn
on the CPU with a fixed seed and moved to HBM before timing.

One step = one routed prefill through the public API, exactly as a caller
runs it: build_switch_query_indices(mask) + switch_gqa_prefill_forward(...)
(compaction with its device-to-host count read, the checks, and the
attention launch; lists fresh from the compaction skip the device index
scan, which any other lists get).  value = routed FLOPs / step time, where
routed FLOPs are counted exactly from the mask (4*d*Hq per legal query/key
pair).

The JSON line also carries:
* roofline: the attention kernel alone, timed with HIP events on the stream it
  runs on, against the 2516.6 TFLOP/s dense bf16 MFMA peak, and beside it the
  rate a register-only MFMA stream holds on this chip (swattn_mfma_peak, a
  probe in its own library, libswattn_probe.so);
  ``traffic`` is copied from the committed rocprofv3 byte-counter summary
  (``traffic_source`` says so), and ``gather_scatter`` is the rate of the
  indexed Q reads and O / LSE writes over the kernel time;
* cpu_baseline: the fp32 PyTorch oracle (a restatement of the reference's
  semantics -- the reference has no CPU path) on a bounded random row sample
  of the same workload, on this host's cores (CPU model stated), and the
  whole config #1 prefill (median of 10 after 2 warm-ups);
* comparators: the same kernel on all-full routing (dense causal), torch
  SDPA causal (flash backend) on the same shape, the compaction alone, the
  routed decode extension (64 sequences, 8192-key caches) against HBM, the
  routed backward (dq, dk, dv) of the same prefill, and one GPU's share of
  the configuration under a KV-head split (Hq4/Hkv1), forward and
  backward, with the fraction of linear scaling 8 such GPUs would give.

``--configs cpu,b2,s16k,varlen,s64k,kvh1`` instead times the forward and the
backward on each named workload (one JSON line each, no roofline);
``--p-sweep 0,0.1,0.25,0.5,1`` times config #3's attention call at each
router density, beside the dense-causal call (one JSON line each); with
``--power`` each call also loops for about 3 s while amd-smi samples the
board power and the shader clock, and so does a register-only MFMA stream.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA (AMD public spec)
PEAK_HBM_GBS = 8000.0
METRIC = "routed-attn TFLOP/s + ms/prefill at S=16k Hq32/Hkv8; % of bf16 MFMA peak"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--p-full", type=float, default=0.25)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="budget for the CPU baseline sample (0 disables it)")
    ap.add_argument("--no-sdpa", action="store_true", help="skip the torch SDPA comparator")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only loop the attention kernel (for rocprofv3 runs)")
    ap.add_argument("--backward-only", action="store_true",
                    help="only loop switch_gqa_prefill_backward (for rocprofv3 runs)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only loop switch_gqa_decode_forward on the decode comparator's "
                         "workload (for rocprofv3 runs)")
    ap.add_argument("--p-sweep", default="",
                    help="comma-separated p_full values: config #3's attention call at each "
                         "router density (e.g. 0,0.1,0.25,0.5,1)")
    ap.add_argument("--power", action="store_true",
                    help="with --p-sweep: also loop each call for about 3 s while sampling the "
                         "board power and the shader clock (amd-smi), and the same for a "
                         "register-only MFMA stream")
    ap.add_argument("--configs", default="",
                    help="comma-separated workloads (cpu,b2,s16k,varlen,s64k): time the "
                         "forward and the backward on each once the clock has settled, one "
                         "JSON line per workload")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="with --kernel-only: also run 3 device copies of this many MiB "
                         "(calibrates the HBM byte counters)")
    return ap.parse_args()


def time_launches(fn, iters, warmup=3):
    """Average ms per call of fn() between two events on torch's current stream."""
    for _ in range(warmup):
        fn()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / iters


def settled_ms(fn, min_iters=10):
    """Average ms per call after about 0.4 s of back-to-back calls (the
    clock rises for tens of milliseconds from idle), over at least 0.3 s."""
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    one = max(time.perf_counter() - t0, 1e-5)
    return time_launches(fn, max(min_iters, int(0.3 / one)), warmup=max(3, int(0.4 / one)))


def config_table(args):
    """Forward and backward of each named workload: routed FLOPs, time and
    rate (backward on the 2.5 x forward-FLOP convention)."""
    from switchattentionkernels_amd import (build_switch_attention_metadata,
                                            build_switch_query_indices, routed_flops,
                                            switch_gqa_prefill_backward,
                                            switch_gqa_prefill_forward, workloads)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    for name in args.configs.split(","):
        wl = workloads.build(name, seed=args.seed)
        q, k, v, m = (wl[x].to(dev) for x in ("q", "k", "v", "mask"))
        W = wl["window"]
        full, local = build_switch_query_indices(m)
        md = None
        if wl["cu_seqlens"] is not None:
            md = build_switch_attention_metadata(q.shape[1], k.shape[1], device=dev, window_size=W,
                                                 cu_seqlens=wl["cu_seqlens"])
        flops = routed_flops(full, local, batch=q.shape[0], seq_q=q.shape[1], seq_kv=k.shape[1],
                             heads_q=q.shape[2], head_dim=128, window=W, metadata=md)

        def fwd():
            return switch_gqa_prefill_forward(q, k, v, full, local, window_size=W, metadata=md)

        f_ms = settled_ms(fwd)
        o, lse = fwd()
        gen = torch.Generator().manual_seed(args.seed + 1)
        do = torch.randn(q.shape, generator=gen).to(torch.bfloat16).to(dev)
        b_ms = settled_ms(lambda: switch_gqa_prefill_backward(q, k, v, o, lse, do, full, local,
                                                              window_size=W, metadata=md))
        print(json.dumps({
            "config": name,
            "shape": f"B{q.shape[0]} S{q.shape[1]} Hq{q.shape[2]}/Hkv{k.shape[2]} W{W}",
            "routed_gflop": round(flops / 1e9, 1),
            "fwd_ms": round(f_ms, 4), "fwd_tflops": round(flops / f_ms / 1e9, 1),
            "fwd_frac_of_peak": round(flops / f_ms / 1e9 / PEAK_BF16_TFLOPS, 4),
            "bwd_ms": round(b_ms, 4), "bwd_tflops_2p5x": round(2.5 * flops / b_ms / 1e9, 1)}),
            flush=True)
        del q, k, v, m, o, lse, do, full, local, md
        torch.cuda.empty_cache()


class PowerSampler:
    """Board power (W) and mean shader clock (MHz) of GPU 0, sampled by
    `amd-smi metric -p -c` in a thread about five times a second."""

    def __init__(self):
        import re
        import shutil
        import subprocess
        import threading
        self._re_p = re.compile(r"SOCKET_POWER:\s*([\d.]+)")
        self._re_c = re.compile(r"GFX_\d+:\s*\n\s*CLK:\s*([\d.]+)")
        self._cmd = ["amd-smi", "metric", "-p", "-c", "-g", "0"]
        self._run = subprocess.run
        self.samples = []
        self._stop = threading.Event()
        self._thread = None
        if shutil.which("amd-smi"):
            self._thread = threading.Thread(target=self._loop, daemon=True)
            self._thread.start()

    def _loop(self):
        while not self._stop.is_set():
            t = time.perf_counter()
            try:
                txt = self._run(self._cmd, capture_output=True, text=True, timeout=5).stdout
            except Exception:  # sampling is diagnostic only
                txt = ""
            pw = self._re_p.search(txt)
            clk = [float(x) for x in self._re_c.findall(txt)]
            if pw and clk:
                self.samples.append((t, float(pw.group(1)), sum(clk) / len(clk)))
            self._stop.wait(0.2)

    def mean(self, t0, t1):
        sel = [(p, c) for t, p, c in self.samples if t0 <= t <= t1]
        if not sel:
            return None, None, 0
        return (round(sum(p for p, _ in sel) / len(sel), 1), round(sum(c for _, c in sel) / len(sel)),
                len(sel))

    def stop(self):
        self._stop.set()
        if self._thread is not None:
            self._thread.join(timeout=10)


def _powered(sampler, fn, seconds=3.0, settle=1.0):
    """Loop fn() for `seconds`; ms per call over the part after `settle`, with
    the mean board power and clock sampled meanwhile."""
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < settle:
        fn()
        torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    s.record()
    n = 0
    while time.perf_counter() - t0 < seconds - settle:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    e.record()
    e.synchronize()
    t1 = time.perf_counter()
    pw, clk, ns = sampler.mean(t0, t1)
    return s.elapsed_time(e) / n, pw, clk, ns


def p_sweep(args):
    """Config #3 (s16k) over router densities: the swattn_prefill_fwd call
    (vt_pack_kernel + the attention kernel) timed on its stream once the clock has
    settled, its routed TFLOP/s and fraction of the bf16 MFMA peak, and its
    time over the same call with every row routed full (dense causal) beside
    the routed-FLOP fraction."""
    from switchattentionkernels_amd import _lib, build_switch_query_indices, routed_flops, workloads
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    dense_ms = None
    sampler = PowerSampler() if args.power else None
    for p in [float(x) for x in args.p_sweep.split(",")]:
        wl = workloads.build("s16k", seed=args.seed, p_full=p)
        d = wl["workload"]
        B, S, HQ, HKV, W = d.batch, d.seq_len, d.heads_q, d.heads_kv, d.window
        q, k, v, m = (wl[x].to(dev) for x in ("q", "k", "v", "mask"))
        out = torch.empty_like(q)
        lse = torch.empty(q.shape[:3], dtype=torch.float32, device=dev)
        ws_bytes = int(L.swattn_prefill_workspace_bytes(B, S, HKV, 128))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        scale = 128 ** -0.5 * 1.4426950408889634

        def attn(fi, li):
            st = L.swattn_prefill_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), fi.data_ptr(),
                                      fi.numel(), li.data_ptr(), li.numel(), None, None, None,
                                      out.data_ptr(), lse.data_ptr(), B, S, S, HQ, HKV, 128, W,
                                      scale, ws.data_ptr(), ws_bytes, stream)
            if st != 0:
                raise RuntimeError(L.swattn_last_error().decode())

        if dense_ms is None:
            fa, la = build_switch_query_indices(torch.ones_like(m))
            dense_ms = settled_ms(lambda: attn(fa, la))
            dense_flops = routed_flops(fa, la, batch=B, seq_q=S, seq_kv=S, heads_q=HQ,
                                       head_dim=128, window=W)
        full, local = build_switch_query_indices(m)
        flops = routed_flops(full, local, batch=B, seq_q=S, seq_kv=S, heads_q=HQ, head_dim=128,
                             window=W)
        ms = settled_ms(lambda: attn(full, local))
        line = {
            "p_sweep": p, "workload": f"s16k: B{B} S{S} Hq{HQ}/Hkv{HKV} d128 W{W} Bernoulli "
                                      f"p_full={p}, seed {args.seed}",
            "full_rows": int(full.numel()), "routed_gflop": round(flops / 1e9, 2),
            "entry_point_ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 1),
            "frac_of_peak": round(flops / ms / 1e9 / PEAK_BF16_TFLOPS, 4),
            "routed_flop_fraction": round(flops / dense_flops, 4),
            "routed_over_dense_time": round(ms / dense_ms, 4), "dense_ms": round(dense_ms, 4)}
        if sampler is not None:
            pms, pw, clk, ns = _powered(sampler, lambda: attn(full, local))
            line.update({"powered_ms": round(pms, 4), "board_power_w": pw, "gfx_clock_mhz": clk,
                         "power_samples": ns})
        print(json.dumps(line), flush=True)
        del q, k, v, m, out, lse, ws, full, local
        torch.cuda.empty_cache()
    if sampler is not None:
        # The same for a register-only MFMA stream (two waves per SIMD).
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        blocks, iters = 2 * cus, 20000
        probe = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
        P = _lib.probe_lib()

        def peak():
            st = P.swattn_mfma_peak(iters, blocks, probe.data_ptr(), stream)
            if st != 0:
                raise RuntimeError(f"swattn_mfma_peak failed with status {st}")

        pms, pw, clk, ns = _powered(sampler, peak)
        print(json.dumps({"power_probe": "register-only bf16 MFMA stream",
                          "tflops": round(blocks * 4 * iters * 8 * 32768 / (pms * 1e-3) / 1e12, 1),
                          "board_power_w": pw, "gfx_clock_mhz": clk, "power_samples": ns}),
              flush=True)
        sampler.stop()


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _cpu_config1(seed: int) -> dict:
    """The CPU timing planned for config #1 (B1 S1024 Hq8/Hkv2 W256, p_full
    0.25): the whole oracle prefill, 2 warm-ups, median of 10."""
    import numpy as np
    import oracle
    from oracle import routing as R
    from switchattentionkernels_amd import workloads
    wl = workloads.build("cpu", seed=seed)
    f_np, l_np = R.compact(wl["mask"].numpy())
    d = wl["workload"]
    i = np.arange(d.seq_len)
    is_full = np.zeros(d.seq_len, dtype=bool)
    is_full[f_np] = True
    pairs = int(np.where(is_full, i + 1, np.minimum(i + 1, d.window)).sum())
    flops = 4 * 128 * d.heads_q * pairs

    def run():
        oracle.routed_attention(wl["q"], wl["k"], wl["v"], f_np, l_np, window_size=d.window)

    times = []
    with torch.inference_mode():
        for it in range(12):
            t0 = time.perf_counter()
            run()
            if it >= 2:
                times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    return {"workload": f"config #1: B1 S{d.seq_len} Hq{d.heads_q}/Hkv{d.heads_kv} d128 "
                        f"W{d.window} p_full={d.p_full}, seed {seed}",
            "ms_median_of_10": round(med * 1e3, 3), "routed_gflop": round(flops / 1e9, 3),
            "gflops": round(flops / med / 1e9, 2), "threads": torch.get_num_threads(),
            "method": "whole fp32 oracle prefill under inference_mode, 2 warm-ups, "
                      "median of 10 (time.perf_counter)"}


def decode_comparator(args, dev, HQ, HKV, D, W, iters, warmup):
    """Routed decode on 64 sequences with 8192-key caches, Bernoulli(p_full)
    routing: time per call and the HBM rate of its algorithmic bytes (the
    routed K and V rows, plus Q and O)."""
    from switchattentionkernels_amd import switch_gqa_decode_forward
    db, dl = 64, 8192
    gen = torch.Generator().manual_seed(args.seed)
    dq = torch.randn(db, 1, HQ, D, generator=gen).to(torch.bfloat16).to(dev)
    dk = torch.randn(db, dl, HKV, D, generator=gen).to(torch.bfloat16).to(dev)
    dv = torch.randn(db, dl, HKV, D, generator=gen).to(torch.bfloat16).to(dev)
    dlens = torch.full((db,), dl, dtype=torch.int32, device=dev)
    dfull = (torch.rand(db, generator=gen) < args.p_full).to(dev)
    dkeys = sum(dl if f else min(dl, W) for f in dfull.tolist())
    dbytes = dkeys * HKV * D * 2 * 2 + 2 * db * HQ * D * 2
    dec_ms = time_launches(lambda: switch_gqa_decode_forward(dq, dk, dv, dlens, dfull,
                                                              window_size=W), iters, warmup=warmup)
    return {"workload": f"B{db} cache {dl} Hq{HQ}/Hkv{HKV} W{W} p_full={args.p_full}, "
                        f"{int(dfull.sum())} full",
            "us": round(dec_ms * 1e3, 1), "hbm_gbs": round(dbytes / (dec_ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(dbytes / (dec_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 3),
            "bytes": dbytes}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                          "(sharding across GPUs is designed, not implemented)"}))
        sys.exit(2)

    if args.configs:
        config_table(args)
        return
    if args.p_sweep:
        p_sweep(args)
        return

    from switchattentionkernels_amd import (build_switch_query_indices, routed_flops,
                                            switch_gqa_prefill_forward, workloads)
    from switchattentionkernels_amd import _lib

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    wl = workloads.build("s16k", seed=args.seed, p_full=args.p_full)
    desc = wl["workload"]
    B, S, HQ, HKV, D, W = desc.batch, desc.seq_len, desc.heads_q, desc.heads_kv, 128, desc.window
    q, k, v = wl["q"].to(dev), wl["k"].to(dev), wl["v"].to(dev)
    mask = wl["mask"].to(dev)
    torch.cuda.synchronize()

    def step():
        full, local = build_switch_query_indices(mask)
        return switch_gqa_prefill_forward(q, k, v, full, local, window_size=W)

    full, local = build_switch_query_indices(mask)
    flops = routed_flops(full, local, batch=B, seq_q=S, seq_kv=S, heads_q=HQ, head_dim=D,
                         window=W)
    dense_flops = 4 * D * HQ * B * S * (S + 1) // 2
    L = _lib.lib()
    scale = D ** -0.5 * 1.4426950408889634
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=dev)
    stream = _lib.stream_handle(dev)
    ws_bytes_fwd = int(L.swattn_prefill_workspace_bytes(B, S, HKV, D))
    ws_fwd = torch.empty(ws_bytes_fwd, dtype=torch.uint8, device=dev)

    def attn(fi, li):
        st = L.swattn_prefill_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), fi.data_ptr(),
                                  fi.numel(), li.data_ptr(), li.numel(), None, None, None,
                                  out.data_ptr(), lse.data_ptr(), B, S, S, HQ, HKV, D, W, scale,
                                  ws_fwd.data_ptr(), ws_bytes_fwd, stream)
        if st != 0:
            raise RuntimeError(L.swattn_last_error().decode())

    if args.kernel_only:
        # The same entry-point launches the roofline figure times, so that a
        # profiler's per-kernel averages over this run can be set beside it.
        kernel_ms = time_launches(lambda: attn(full, local), args.steps, warmup=args.warmup)
        # Calibration for HBM byte counters: a plain device-to-device copy of
        # a known size (its FETCH_SIZE / WRITE_SIZE per dispatch, divided by
        # these bytes, is the counter's scale factor).
        calib = None
        if args.calib_copy_mib > 0:
            n = args.calib_copy_mib << 20
            src = torch.ones(n, dtype=torch.uint8, device=dev)
            dst = torch.empty_like(src)
            for _ in range(3):
                dst.copy_(src)
            torch.cuda.synchronize()
            calib = {"copy_bytes_read": n, "copy_bytes_written": n, "copies": 3}
        print(json.dumps({"kernel_only": True, "launches": args.warmup + args.steps,
                          "timed_launches": args.steps, "entry_point_ms": round(kernel_ms, 4),
                          "calibration": calib}))
        return

    if args.decode_only:
        res = decode_comparator(args, dev, HQ, HKV, D, W, args.steps, args.warmup)
        print(json.dumps({"decode_only": True, "launches": args.warmup + args.steps,
                          "timed_launches": args.steps, **res}))
        return

    if args.backward_only:
        from switchattentionkernels_amd import switch_gqa_prefill_backward
        gen = torch.Generator().manual_seed(args.seed + 1)
        dout = torch.randn(q.shape, generator=gen).to(torch.bfloat16).to(dev)
        o_f, lse_f = switch_gqa_prefill_forward(q, k, v, full, local, window_size=W)
        bwd_ms = time_launches(lambda: switch_gqa_prefill_backward(q, k, v, o_f, lse_f, dout, full,
                                                                   local, window_size=W),
                               args.steps, warmup=args.warmup)
        print(json.dumps({"backward_only": True, "launches": args.warmup + args.steps,
                          "timed_launches": args.steps, "entry_point_ms": round(bwd_ms, 4),
                          "tflops_2p5x": round(2.5 * flops / (bwd_ms * 1e-3) / 1e12, 1)}))
        return

    # ---- attention kernel alone (roofline) -------------------------------------
    # Timed first, after about 0.4 s of untimed calls: they bring the chip from
    # idle to the clock it holds under this load (200 calls after only 10
    # warm-ups measured 1.4 % slower than after the clock settled), and they
    # leave it there for the timed steps below.
    attn(full, local)
    torch.cuda.synchronize()
    t_one = time.perf_counter()
    attn(full, local)
    torch.cuda.synchronize()
    attn_warm = max(10, int(0.4 / max(time.perf_counter() - t_one, 1e-5)))
    attn_calls = max(args.steps, 50)
    attn_ms = time_launches(lambda: attn(full, local), attn_calls, warmup=attn_warm)
    attn_tflops = flops / (attn_ms * 1e-3) / 1e12

    # ---- timed region: K full steps -------------------------------------------
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    print(f"[bench] {args.steps} steps, {ms_step:.3f} ms/step", file=sys.stderr, flush=True)
    ones = torch.ones_like(mask)
    f_all, l_all = build_switch_query_indices(ones)
    dense_ms = time_launches(lambda: attn(f_all, l_all), max(args.steps, 20), warmup=5)
    ws_bytes = int(L.swattn_compact_workspace_bytes(S * B))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    idx = torch.empty(S * B, dtype=torch.int32, device=dev)
    cnt = torch.empty(2, dtype=torch.int32, device=dev)
    compact_ms = time_launches(lambda: L.swattn_compact(mask.data_ptr(), S * B, idx.data_ptr(),
                                                        cnt.data_ptr(), ws.data_ptr(), ws_bytes,
                                                        stream), 50)
    compact_bytes = S * B + 4 * S * B + 8
    # The fused router step (extension): bf16 logits > 0 compacted in one pass.
    logits = torch.randn(S * B, generator=torch.Generator().manual_seed(args.seed + 2))
    logits = logits.to(torch.bfloat16).to(dev)
    logits_ms = time_launches(lambda: L.swattn_compact_logits(
        logits.data_ptr(), 1, S * B, 0.0, idx.data_ptr(), cnt.data_ptr(), ws.data_ptr(),
        ws_bytes, stream), 50)
    # The split-key merge (extension): two partial (O, LSE) pairs of this
    # prefill's shape folded into one; HBM bytes = 2 partials in, 1 out.
    from switchattentionkernels_amd import merge_attention_partials
    lse_b = lse.clone()
    merge_ms = time_launches(lambda: merge_attention_partials([out, out], [lse, lse_b]), 20)
    merge_bytes = 3 * (out.numel() * 2 + lse.numel() * 4)
    del lse_b
    print(f"[bench] attention kernel {attn_ms:.3f} ms ({attn_tflops:.1f} TFLOP/s); dense causal "
          f"{dense_ms:.3f} ms; compaction {compact_ms * 1e3:.1f} us", file=sys.stderr, flush=True)

    # ---- achievable MFMA rate: register-only bf16 MFMA stream, two waves per SIMD ----
    mfma_tflops = None
    try:
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        blocks, iters = 2 * cus, 20000
        probe = torch.empty(blocks * 256, dtype=torch.float32, device=dev)

        P = _lib.probe_lib()

        def peak():
            st = P.swattn_mfma_peak(iters, blocks, probe.data_ptr(), stream)
            if st != 0:
                raise RuntimeError(f"swattn_mfma_peak failed with status {st}")

        peak_ms = time_launches(peak, 5, warmup=2)
        mfma_tflops = blocks * 4 * iters * 8 * 32768 / (peak_ms * 1e-3) / 1e12
        print(f"[bench] MFMA-only probe {mfma_tflops:.1f} TFLOP/s", file=sys.stderr, flush=True)
    except Exception as exc:  # diagnostic only
        print(f"[bench] MFMA probe unavailable: {exc}", file=sys.stderr, flush=True)

    # ---- SDPA comparator (flash backend, GQA expanded) -------------------------
    sdpa_ms = None
    if not args.no_sdpa:
        try:
            from torch.nn.attention import SDPBackend, sdpa_kernel
            g = HQ // HKV
            qt = q.permute(0, 2, 1, 3).contiguous()
            kt = k.repeat_interleave(g, dim=2).permute(0, 2, 1, 3).contiguous()
            vt = v.repeat_interleave(g, dim=2).permute(0, 2, 1, 3).contiguous()
            with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
                sdpa_ms = time_launches(lambda: torch.nn.functional.scaled_dot_product_attention(
                    qt, kt, vt, is_causal=True), 5, warmup=2)
            del qt, kt, vt
        except Exception as exc:  # comparator only
            print(f"[bench] SDPA comparator unavailable: {exc}", file=sys.stderr, flush=True)

    # ---- routed decode (extension): one token per sequence over its KV cache ------
    decode = None
    try:
        decode = decode_comparator(args, dev, HQ, HKV, D, W, 20, 5)
    except Exception as exc:  # comparator only
        print(f"[bench] decode comparator unavailable: {exc}", file=sys.stderr, flush=True)

    # ---- routed backward (extension): dq, dk, dv of the same prefill --------------
    backward = None
    try:
        from switchattentionkernels_amd import switch_gqa_prefill_backward
        gen = torch.Generator().manual_seed(args.seed + 1)
        dout = torch.randn(q.shape, generator=gen).to(torch.bfloat16).to(dev)
        o_f, lse_f = switch_gqa_prefill_forward(q, k, v, full, local, window_size=W)
        # Timed like the forward kernel: back-to-back calls once the clock
        # has settled (the first calls after idle run at another clock).
        bwd_ms = settled_ms(lambda: switch_gqa_prefill_backward(q, k, v, o_f, lse_f, dout, full,
                                                                local, window_size=W))
        # Five products per legal (row, key) pair (S, dP, dV, dK, dQ): 2.5x
        # the forward's two; the dQ pass recomputes S and dP on top of that.
        backward = {"ms": round(bwd_ms, 4), "tflops": round(2.5 * flops / (bwd_ms * 1e-3) / 1e12, 1),
                    "flop_convention": "2.5 x routed forward FLOPs",
                    "frac_of_peak": round(2.5 * flops / (bwd_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                    "timing": "HIP events around back-to-back calls after about 0.4 s of untimed "
                              "calls (clock settled)"}
        print(f"[bench] backward {bwd_ms:.3f} ms ({backward['tflops']} TFLOP/s)", file=sys.stderr,
              flush=True)
        del dout, o_f, lse_f
    except Exception as exc:  # comparator only
        print(f"[bench] backward comparator unavailable: {exc}", file=sys.stderr, flush=True)

    # ---- one GPU's share under a KV-head split (the sharding design) -------------
    # Hkv / 8 KV heads with their query heads: what each of 8 GPUs would run,
    # timed on this one, forward and backward; "linear" is 8 x that share's
    # time against the whole configuration's on one GPU, both sides timed
    # alike: the public API call, settled.
    kv_share = None
    try:
        from switchattentionkernels_amd import switch_gqa_prefill_backward
        f_whole = settled_ms(lambda: switch_gqa_prefill_forward(q, k, v, full, local, window_size=W))
        o_w, lse_w = switch_gqa_prefill_forward(q, k, v, full, local, window_size=W)
        do_w = torch.randn(q.shape, generator=torch.Generator().manual_seed(args.seed + 1))
        do_w = do_w.to(torch.bfloat16).to(dev)
        b_whole = settled_ms(lambda: switch_gqa_prefill_backward(q, k, v, o_w, lse_w, do_w, full,
                                                                 local, window_size=W))
        del o_w, lse_w, do_w
        wl_s = workloads.build("kvh1", seed=args.seed)
        qs, ks, vs, ms = (wl_s[x].to(dev) for x in ("q", "k", "v", "mask"))
        ws_ = wl_s["window"]
        fs, ls = build_switch_query_indices(ms)
        f_share = settled_ms(lambda: switch_gqa_prefill_forward(qs, ks, vs, fs, ls, window_size=ws_))
        o_s, lse_s = switch_gqa_prefill_forward(qs, ks, vs, fs, ls, window_size=ws_)
        do_s = torch.randn(qs.shape, generator=torch.Generator().manual_seed(args.seed + 2))
        do_s = do_s.to(torch.bfloat16).to(dev)
        b_share = settled_ms(lambda: switch_gqa_prefill_backward(qs, ks, vs, o_s, lse_s, do_s, fs,
                                                                 ls, window_size=ws_))
        kv_share = {"workload": f"kvh1: B1 S{qs.shape[1]} Hq{qs.shape[2]}/Hkv{ks.shape[2]} W{ws_}, "
                                f"Bernoulli(0.25), seed {args.seed}",
                    "fwd_ms": round(f_share, 4),
                    "whole_fwd_ms": round(f_whole, 4),
                    "fwd_linear_frac": round(f_whole / (8 * f_share), 3),
                    "bwd_ms": round(b_share, 4),
                    "whole_bwd_ms": round(b_whole, 4),
                    "bwd_linear_frac": round(b_whole / (8 * b_share), 3)}
        del qs, ks, vs, ms, fs, ls, o_s, lse_s, do_s
    except Exception as exc:  # comparator only
        print(f"[bench] KV-head share comparator unavailable: {exc}", file=sys.stderr, flush=True)

    # ---- traffic: copied from the committed rocprofv3 --pmc summary, if any ------
    # (byte counters cannot be read inside this timed run; the file states the
    # command and the calibration that produced the figure)
    traffic, traffic_src = None, None
    tpath = os.path.join(ROOT, "profiles", "fwd_s16k_p25_traffic.txt")
    if os.path.exists(tpath):
        for line in open(tpath):
            if line.startswith("traffic_bytes_per_launch"):
                traffic = int(float(line.split("=")[1]))
                traffic_src = ("copied from profiles/fwd_s16k_p25_traffic.txt (rocprofv3 --pmc "
                               "FETCH_SIZE + WRITE_SIZE per launch, calibrated by a device copy); "
                               "not measured in this run")

    # ---- gather / scatter: Q rows read by index, O and LSE rows written by index ----
    rows = B * S
    gather_scatter_bytes = rows * HQ * D * 2 + rows * HQ * D * 2 + rows * HQ * 4 + rows * 4

    # ---- CPU baseline: the oracle on a bounded row sample -------------------------
    cpu = None
    if args.cpu_seconds > 0:
        cpu_model = _cpu_model()
        config1 = _cpu_config1(args.seed)
        import numpy as np
        import oracle
        from oracle import routing as R
        f_np, l_np = R.compact(wl["mask"].numpy())
        chunk = 256
        blocks = torch.randperm((B * S) // chunk,
                                generator=torch.Generator().manual_seed(1)).tolist()
        done, t_cpu = [], 0.0
        with torch.inference_mode():
            oracle.routed_attention(wl["q"], wl["k"], wl["v"], f_np, l_np, window_size=W,
                                    rows=np.arange(chunk))   # warm-up
            for blk in blocks:
                if t_cpu >= args.cpu_seconds:
                    break
                r = np.arange(blk * chunk, (blk + 1) * chunk)
                t1 = time.perf_counter()
                oracle.routed_attention(wl["q"], wl["k"], wl["v"], f_np, l_np, window_size=W,
                                        rows=r)
                t_cpu += time.perf_counter() - t1
                done.append(r)
        sample = np.concatenate(done)
        rows_done = sample.size
        is_full = np.zeros(B * S, dtype=bool)
        is_full[f_np] = True
        i = sample % S
        pairs = np.where(is_full[sample], i + 1, np.minimum(i + 1, W)).sum()
        cpu_flops = 4 * D * HQ * int(pairs)
        cpu = {"value": round(cpu_flops / t_cpu / 1e12, 4), "unit": "TFLOP/s",
               "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"{rows_done} query rows (all {HQ} heads) in {len(done)} random "
                         f"{chunk}-row blocks of the s16k p_full="
                         f"{args.p_full} workload, fp32 dense-masked torch oracle, "
                         f"{t_cpu:.1f} s; host {os.cpu_count()} cpus, affinity "
                         f"{len(os.sched_getaffinity(0))}",
               "cpu_model": cpu_model,
               "ms_per_prefill_extrapolated": round(t_cpu * 1e3 * B * S / rows_done, 1),
               "config1": config1}

    achieved = attn_tflops
    res = {
        "metric": METRIC,
        "value": round(flops / (ms_step * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded bf16 N(0,1) Q/K/V, Bernoulli route mask)",
        "config": {"workload": f"s16k: B{B} S{S} Hq{HQ}/Hkv{HKV} d{D} W{W} "
                               f"p_full={args.p_full} Bernoulli, seed {args.seed}",
                   "batch": B, "seq_len": S, "heads_q": HQ, "heads_kv": HKV, "head_dim": D,
                   "window": W, "p_full": args.p_full, "routed_gflop": round(flops / 1e9, 2)},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": ("swattn_prefill_fwd: vt_pack_kernel + fwd_wide_kernel<false> (the "
                                "256-row kernel, which swattn_prefill_fwd picks at this grid size)"),
                     "kernel_ms": round(attn_ms, 4),
                     "kernel_timing": f"HIP events on the launch stream around "
                                      f"{attn_calls} back-to-back calls after {attn_warm} "
                                      f"untimed calls (about 0.4 s: clock settled), in this "
                                      f"run",
                     "gather_scatter": {
                         "bytes": gather_scatter_bytes,
                         "what": "Q rows read and O / LSE rows written at their listed "
                                 "positions, plus the index lists, over the kernel time",
                         "gbs": round(gather_scatter_bytes / (attn_ms * 1e-3) / 1e9, 1),
                         "hbm_frac": round(gather_scatter_bytes / (attn_ms * 1e-3) / 1e9
                                           / PEAK_HBM_GBS, 4)},
                     "achievable_mfma_tflops": None if mfma_tflops is None
                     else round(mfma_tflops, 1),
                     "frac_of_achievable": None if mfma_tflops is None
                     else round(achieved / mfma_tflops, 4)},
        "cpu_baseline": cpu,
        "comparators": {
            "dense_causal_same_kernel_ms": round(dense_ms, 4),
            "routed_flop_fraction": round(flops / dense_flops, 4),
            "routed_over_dense_time": round(attn_ms / dense_ms, 4),
            "sdpa_flash_causal_ms": None if sdpa_ms is None else round(sdpa_ms, 4),
            "routed_over_sdpa_dense_time": None if sdpa_ms is None
            else round(attn_ms / sdpa_ms, 4),
            "compaction_us": round(compact_ms * 1e3, 2),
            "compaction_gbs": round(compact_bytes / (compact_ms * 1e-3) / 1e9, 1),
            "compaction_logits_us": round(logits_ms * 1e3, 2),
            "merge_two_partials_us": round(merge_ms * 1e3, 1),
            "merge_hbm_gbs": round(merge_bytes / (merge_ms * 1e-3) / 1e9, 1),
            "decode": decode,
            "backward": backward,
            "kv_head_share": kv_share,
        },
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
