"""Seeded synthetic workloads for the routed prefill.

The reference has no router (README:85, V:309-310): a model produces a hard
``bool`` mask per token.  These generators stand in for it in tests and the
benchmark.  Every tensor is drawn on the CPU from ``torch.Generator`` with a
fixed seed, so CPU and GPU runs see identical bf16 inputs.

Configurations (head_dim 128 throughout):

=====  ==========================================================  =========
name   shape                                                       routing
=====  ==========================================================  =========
cpu    B1  S1024  Hq8/Hkv2   W256                                   Bernoulli(0.25)
b2     B2  S4096  Hq32/Hkv8  W1024, inputs x0.5                      Bernoulli(p), p in {0, .25, 1}
s16k   B1  S16384 Hq32/Hkv8  W1024                                  Bernoulli(p), p in {.1, .25, .5}
varlen 8 seqs, lengths U[512, 8192], Hq64/Hkv8, W2048               Markov(stay .95, p .3)
s64k   B1  S65536 Hq40/Hkv8  W4096                                  ramp 0.05 -> 0.25
kvh1   B1  S16384 Hq4/Hkv1   W1024 (one GPU's share of s16k split   Bernoulli(0.25)
       by KV head over 8 GPUs)
=====  ==========================================================  =========
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass
class Workload:
    name: str
    batch: int
    seq_len: int
    heads_q: int
    heads_kv: int
    window: int
    head_dim: int = 128
    scale: float = 1.0
    routing: str = "bernoulli"
    p_full: float = 0.25
    cu_seqlens: list | None = None
    extra: dict = field(default_factory=dict)


CONFIGS = {
    "cpu": Workload("cpu", 1, 1024, 8, 2, 256),
    "b2": Workload("b2", 2, 4096, 32, 8, 1024, scale=0.5),
    "s16k": Workload("s16k", 1, 16384, 32, 8, 1024),
    "varlen": Workload("varlen", 1, 0, 64, 8, 2048, routing="markov", p_full=0.3),
    "s64k": Workload("s64k", 1, 65536, 40, 8, 4096, routing="ramp", p_full=0.15),
    "kvh1": Workload("kvh1", 1, 16384, 4, 1, 1024),
}


def bernoulli_mask(gen: torch.Generator, shape, p: float) -> torch.Tensor:
    """i.i.d. Bernoulli(p) route per token (True = full)."""
    return torch.rand(shape, generator=gen) < p


def markov_mask(gen: torch.Generator, length: int, p: float, stay: float = 0.95) -> torch.Tensor:
    """Clustered routing: keep the previous state with probability ``stay``,
    otherwise redraw from Bernoulli(p).  The first state is Bernoulli(p), so the
    stationary full fraction is exactly ``p`` and runs are contiguous."""
    u = torch.rand(length, generator=gen)
    redraw = torch.rand(length, generator=gen) < p
    out = torch.empty(length, dtype=torch.bool)
    state = bool(redraw[0])
    keep = (u >= 1.0 - stay).tolist()
    rd = redraw.tolist()
    for i in range(length):
        if i > 0 and not keep[i]:
            state = rd[i]
        out[i] = state
    return out


def ramp_mask(gen: torch.Generator, length: int, lo: float = 0.05, hi: float = 0.25) -> torch.Tensor:
    """Full-routing probability ramping linearly from ``lo`` to ``hi``."""
    p = torch.linspace(lo, hi, length)
    return torch.rand(length, generator=gen) < p


def varlen_lengths(gen: torch.Generator, nseq: int = 8, lo: int = 512, hi: int = 8192) -> list:
    return torch.randint(lo, hi + 1, (nseq,), generator=gen).tolist()


def make_qkv(gen: torch.Generator, batch, seq_q, seq_kv, hq, hkv, d=128, scale=1.0):
    """bf16 Q/K/V drawn as fp32 N(0,1) * scale, then rounded to bf16 (CPU)."""
    q = (torch.randn(batch, seq_q, hq, d, generator=gen) * scale).to(torch.bfloat16)
    k = (torch.randn(batch, seq_kv, hkv, d, generator=gen) * scale).to(torch.bfloat16)
    v = (torch.randn(batch, seq_kv, hkv, d, generator=gen) * scale).to(torch.bfloat16)
    return q, k, v


def build(name: str, seed: int = 0, p_full: float | None = None, **overrides):
    """Materialise a named workload on the CPU.

    Returns a dict with ``q, k, v`` (bf16 CPU tensors), ``mask`` (bool, shape
    ``[B, S]``), ``window``, ``cu_seqlens`` (int32 list or None) and the
    ``Workload`` description.
    """
    wl = CONFIGS[name]
    wl = Workload(**{**wl.__dict__, **overrides})
    if p_full is not None:
        wl.p_full = p_full
    gen = torch.Generator().manual_seed(seed)
    cu = None
    if wl.routing == "markov":
        lens = varlen_lengths(gen)
        cu = [0]
        for n in lens:
            cu.append(cu[-1] + n)
        seq = cu[-1]
        mask = torch.cat([markov_mask(gen, n, wl.p_full) for n in lens])[None]
    elif wl.routing == "ramp":
        seq = wl.seq_len
        mask = ramp_mask(gen, seq)[None]
    else:
        seq = wl.seq_len
        mask = bernoulli_mask(gen, (wl.batch, seq), wl.p_full)
    q, k, v = make_qkv(gen, wl.batch, seq, seq, wl.heads_q, wl.heads_kv, wl.head_dim, wl.scale)
    wl.seq_len = seq
    wl.cu_seqlens = cu
    return {"q": q, "k": k, "v": v, "mask": mask, "window": wl.window,
            "cu_seqlens": cu, "workload": wl}
