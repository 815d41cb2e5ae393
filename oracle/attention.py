"""Floating-point side of the Switch Attention oracle.

TEST INFRASTRUCTURE ONLY -- see the package docstring.  Reference file tags:
V = swiattn_gqa_prefill_varlen.py, F = swiattn_gqa_prefill.py.

Semantics restated (V:103-249):
* each query row q, for every query head h, attends to the keys
  ``[start(q), end(q))`` of KV head ``h // (Hq // Hkv)`` (V:124, V:186-196);
  ``start`` is the row's full or local start depending on its route;
* scores are ``q . k`` scaled by ``sm_scale`` (default ``D**-0.5``, V:73-76);
* ``O = softmax(scores) @ V`` and ``LSE = logsumexp(scores) * log2(e)``
  (log2 convention, V:236-241);
* rows are written back to their own positions (V:243-249).

``routed_attention_backward`` is the derivative of that forward (the reference
itself is forward-only, V:14-15).

The restatement is a dense masked computation in fp32 on the CPU -- no online
softmax, no bf16 rounding of P -- so it is the exact-arithmetic target that
the kernels are compared against within a tolerance.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from .routing import default_bounds

LOG2E = 1.4426950408889634


def row_bounds(full_idx, local_idx, full_starts, local_starts, ends):
    """Per-row ``[start, end)`` for a routed sequence (V:134-137).

    Rows in ``full_idx`` take ``full_starts``, rows in ``local_idx`` take
    ``local_starts``; every row takes ``ends``.
    """
    n = np.asarray(ends).size
    start = np.full(n, -1, dtype=np.int64)
    fi = np.asarray(full_idx, dtype=np.int64).reshape(-1)
    li = np.asarray(local_idx, dtype=np.int64).reshape(-1)
    start[fi] = np.asarray(full_starts, dtype=np.int64)[fi]
    start[li] = np.asarray(local_starts, dtype=np.int64)[li]
    return start, np.asarray(ends, dtype=np.int64).copy()


def _bounds_for(q, k, full_idx, local_idx, window_size, metadata):
    batch, seq_q = int(q.shape[0]), int(q.shape[1])
    seq_kv = int(k.shape[1])
    if metadata is None:
        fs, ls, en = default_bounds(batch, seq_q, seq_kv, window_size)
    else:
        fs = np.asarray(metadata["full_starts"], dtype=np.int64)
        ls = np.asarray(metadata["local_starts"], dtype=np.int64)
        en = np.asarray(metadata["causal_ends"], dtype=np.int64)
    start, end = row_bounds(full_idx, local_idx, fs, ls, en)
    total_kv = batch * seq_kv
    return np.clip(start, 0, total_kv), np.clip(end, 0, total_kv)


def routed_attention(q, k, v, full_idx, local_idx, *, window_size=1024,
                     metadata=None, sm_scale=None, rows=None, chunk=256):
    """Dense masked routed attention in fp32.

    q: ``[B, Sq, Hq, D]``, k/v: ``[B, Skv, Hkv, D]`` (any float dtype, CPU).
    ``full_idx``/``local_idx`` are flattened row positions ``b*Sq + i``.
    ``metadata`` (optional) is a dict with ``full_starts``, ``local_starts``,
    ``causal_ends`` in flattened key coordinates.  ``rows`` (optional) limits
    the computation to a subset of flattened rows (for bounded timing samples).

    Returns ``(O fp32 [B, Sq, Hq, D], LSE fp32 [B, Sq, Hq])``; rows outside
    ``rows`` are left NaN.
    """
    batch, seq_q, hq, d = (int(x) for x in q.shape)
    hkv = int(k.shape[2])
    g = hq // hkv
    scale = (1.0 / d) ** 0.5 if sm_scale is None else float(sm_scale)
    start, end = _bounds_for(q, k, full_idx, local_idx, window_size, metadata)
    qf = q.reshape(batch * seq_q, hq, d).float()
    kf = k.reshape(-1, hkv, d).float()
    vf = v.reshape(-1, hkv, d).float()
    out = torch.full((batch * seq_q, hq, d), float("nan"), dtype=torch.float32)
    lse = torch.full((batch * seq_q, hq), float("nan"), dtype=torch.float32)
    all_rows = np.arange(batch * seq_q) if rows is None else np.asarray(rows)
    for c0 in range(0, all_rows.size, chunk):
        r = all_rows[c0:c0 + chunk]
        ks, ke = int(start[r].min()), int(end[r].max())
        ke = max(ke, ks)
        span = torch.arange(ks, ke)
        legal = (span[None, :] >= torch.from_numpy(start[r])[:, None]) & \
                (span[None, :] < torch.from_numpy(end[r])[:, None])          # [R, L]
        qr = qf[torch.from_numpy(r)].reshape(len(r), hkv, g, d)             # [R, Hkv, G, D]
        qr = qr.permute(1, 0, 2, 3).reshape(hkv, len(r) * g, d)             # [Hkv, R*G, D]
        kt = kf[ks:ke].permute(1, 2, 0).contiguous()                        # [Hkv, D, L]
        s = torch.bmm(qr, kt).reshape(hkv, len(r), g, ke - ks) * scale      # [Hkv, R, G, L]
        s = s.masked_fill(~legal[None, :, None, :], float("-inf"))
        lse_nat = torch.logsumexp(s, dim=-1)                                # [Hkv, R, G]
        p = torch.exp(s - lse_nat[..., None])
        o = torch.bmm(p.reshape(hkv, len(r) * g, ke - ks),
                      vf[ks:ke].permute(1, 0, 2).contiguous())              # [Hkv, R*G, D]
        o = o.reshape(hkv, len(r), g, d).permute(1, 0, 2, 3).reshape(len(r), hq, d)
        lse_r = (lse_nat * LOG2E).permute(1, 0, 2).reshape(len(r), hq)
        # A row with no legal key is 0 / 0 = NaN (V:236-241), also when every
        # row of the chunk is empty and the contraction over no key gives 0.
        o = o.masked_fill(torch.isneginf(lse_r)[..., None], float("nan"))
        out[torch.from_numpy(r)] = o
        lse[torch.from_numpy(r)] = lse_r
    return out.reshape(batch, seq_q, hq, d), lse.reshape(batch, seq_q, hq)


def brute_force_attention(q, k, v, full_mask, window_size, *, cu_seqlens=None,
                          sm_scale=None):
    """Float64 pure-Python routed attention for tiny inputs.

    Written from the definitions alone, independent of ``row_bounds``:
    query i of a sequence may see key j of the same sequence iff ``j <= i``
    (and ``j`` exists), and, when i is routed local, also ``i - j < W``
    (F:145-155).  ``q``/``k``/``v`` are ``[B, S, H, D]`` arrays (converted to
    float64); ``full_mask`` is ``[B, S]`` bool; ``cu_seqlens`` (B must be 1)
    packs several sequences into the single batch row.
    Returns (O ``[B, Sq, Hq, D]``, LSE2 ``[B, Sq, Hq]``) as float64 numpy.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    fm = np.asarray(full_mask, dtype=bool).reshape(q.shape[0], q.shape[1])
    batch, seq_q, hq, d = q.shape
    seq_kv, hkv = k.shape[1], k.shape[2]
    g = hq // hkv
    scale = (1.0 / d) ** 0.5 if sm_scale is None else float(sm_scale)
    if cu_seqlens is None:
        segs = [(0, seq_q, 0, seq_kv)]
    else:
        cu = [int(x) for x in cu_seqlens]
        segs = [(cu[s], cu[s + 1], cu[s], cu[s + 1]) for s in range(len(cu) - 1)]
    out = np.full((batch, seq_q, hq, d), np.nan)
    lse = np.full((batch, seq_q, hq), np.nan)
    for b in range(batch):
        for (q0, q1, k0, k1) in segs:
            for i in range(q1 - q0):
                for h in range(hq):
                    keys = [j for j in range(k1 - k0)
                            if j <= i and (fm[b, q0 + i] or i - j < window_size)]
                    if not keys:
                        continue
                    qi = q[b, q0 + i, h]
                    sc = [scale * float(np.dot(qi, k[b, k0 + j, h // g])) for j in keys]
                    mx = max(sc)
                    w = [math.exp(x - mx) for x in sc]
                    tot = sum(w)
                    acc = np.zeros(d)
                    for wj, j in zip(w, keys):
                        acc += wj * v[b, k0 + j, h // g]
                    out[b, q0 + i, h] = acc / tot
                    lse[b, q0 + i, h] = (mx + math.log(tot)) * LOG2E
    return out, lse


def routed_flops(full_idx, local_idx, batch, seq_q, seq_kv, heads_q, head_dim,
                 window_size, metadata=None) -> int:
    """Algorithmic FLOPs of a routed prefill: ``4 * D * Hq * sum_rows |legal keys|``.

    Two GEMMs (QK^T and PV) of ``2 * D`` FLOPs per legal (row, key, head).
    Softmax work is not counted.
    """
    if metadata is None:
        fs, ls, en = default_bounds(batch, seq_q, seq_kv, window_size)
    else:
        fs, ls, en = (np.asarray(metadata[n], dtype=np.int64)
                      for n in ("full_starts", "local_starts", "causal_ends"))
    start, end = row_bounds(full_idx, local_idx, fs, ls, en)
    pairs = np.maximum(end - start, 0).sum()
    return int(4 * head_dim * heads_q * int(pairs))


def merge_partials(outputs, lses):
    """Combine attention results over disjoint key ranges (float64).

    ``outputs[i]``: ``[..., D]``; ``lses[i]``: ``[...]``, log2 convention
    (V:236-241: LSE = log2 sum_j 2^(s_j c)).  The union's LSE is
    ``log2 sum_i 2^LSE_i`` and its output ``sum_i 2^(LSE_i - LSE) O_i``.
    Parts with LSE = -inf (no legal key) carry no weight; a row empty in every
    part gives NaN / -inf, as an empty row does in ``routed_attention``.
    """
    O = [torch.as_tensor(o, dtype=torch.float64) for o in outputs]
    L = [torch.as_tensor(l, dtype=torch.float64) for l in lses]
    m = torch.stack(L).amax(0)
    live = torch.isfinite(m)
    safe_m = torch.where(live, m, torch.zeros_like(m))
    w = [torch.where(torch.isfinite(l), torch.exp2(l - safe_m), torch.zeros_like(l)) for l in L]
    wsum = sum(w)
    acc = sum(wi.unsqueeze(-1) * torch.nan_to_num(oi) for wi, oi in zip(w, O))
    out = acc / wsum.unsqueeze(-1)
    lse = torch.where(live, safe_m + torch.log2(wsum), torch.full_like(m, -math.inf))
    return out, lse


def decode_attention(q, k_cache, v_cache, cache_lens, full_mask, *, window_size=1024,
                     sm_scale=None):
    """Routed decode in fp32: the prefill rule (F:145-155) for the last row.

    ``q``: ``[B, Hq, D]``; caches ``[B, L, Hkv, D]``; ``cache_lens`` ``[B]``
    (clamped to ``[0, L]``); ``full_mask`` ``[B]`` bool.  The token of sequence
    b sits at position ``n - 1`` (``n = cache_lens[b]``) and sees keys
    ``[0, n)`` when full, else ``[max(n - W, 0), n)``.  Returns
    (O ``[B, Hq, D]``, LSE2 ``[B, Hq]``); a sequence with no key gives NaN /
    -inf.
    """
    q = torch.as_tensor(q).float()
    k = torch.as_tensor(k_cache).float()
    v = torch.as_tensor(v_cache).float()
    batch, hq, d = q.shape
    cache_len, hkv = k.shape[1], k.shape[2]
    g = hq // hkv
    scale = (1.0 / d) ** 0.5 if sm_scale is None else float(sm_scale)
    out = torch.full((batch, hq, d), math.nan)
    lse = torch.full((batch, hq), -math.inf)
    for b in range(batch):
        n = max(0, min(int(cache_lens[b]), cache_len))
        lo = 0 if bool(full_mask[b]) else max(n - window_size, 0)
        if n <= lo:
            continue
        kk = k[b, lo:n].repeat_interleave(g, dim=1)   # [keys, Hq, D]
        vv = v[b, lo:n].repeat_interleave(g, dim=1)
        s = torch.einsum("hd,khd->hk", q[b], kk) * scale
        lse[b] = torch.logsumexp(s, dim=1) * LOG2E
        out[b] = torch.einsum("hk,khd->hd", torch.softmax(s, dim=1), vv)
    return out, lse


def _score_grad(p, dp, delta=None):
    """dS = P * (dP - Delta): the softmax Jacobian applied to dP, with
    Delta = rowsum(P * dP) unless a per-row Delta is given."""
    if delta is None:
        delta = (p * dp).sum(-1, keepdim=True)
    return p * (dp - delta)


def delta_shift_bound(out_used, out_exact, grad_out, pk, scale):
    """Per-row size of the dq change that the FlashAttention-2 Delta brings.

    A backward that takes ``Delta_r = dO_r . out_r`` from a rounded forward
    output ``out`` instead of the exact ``dO_r . O_r`` computes, in exact
    arithmetic otherwise, ``dq_r - scale * delta_r * sum_j P_rj k_j`` with
    ``delta_r = dO_r . (out_r - O_r)`` (see ``routed_attention_backward``).
    Returns ``scale * |delta_r| * ||sum_j P_rj k_j||_2`` per flattened row
    and query head, ``[T, Hq]`` in float64, from the forward output the
    backward used, the exact one, ``dO`` and the ``"pk"`` term that
    ``routed_attention_backward(..., delta_terms=...)`` records.
    """
    hq, d = int(grad_out.shape[-2]), int(grad_out.shape[-1])
    do = grad_out.reshape(-1, hq, d).double()
    diff = out_used.reshape(-1, hq, d).double() - out_exact.reshape(-1, hq, d).double()
    delta = (do * diff).sum(-1)
    return float(scale) * delta.abs() * pk.reshape(-1, hq, d).double().norm(dim=-1)


def routed_attention_backward(q, k, v, grad_out, full_idx, local_idx, *, window_size=1024,
                              metadata=None, sm_scale=None, chunk=256, dtype=torch.float32,
                              rows=None, out=None, delta_terms=None):
    """Gradients of the routed attention output, dense and masked, in ``dtype``.

    The reference is forward-only (V:14-15); this is the derivative of the
    forward restated in ``routed_attention`` (V:103-249) with respect to q, k
    and v, for a loss whose gradient with respect to O is ``grad_out``:

    * ``P = softmax(scale * q.k)`` over each row's legal keys (0 elsewhere),
      ``dP = dO . v``, ``Delta = rowsum(P * dP)``, ``dS = P * (dP - Delta)``;
    * ``dq = scale * dS k``, ``dk = scale * dS^T q``, ``dv = P^T dO``, the last
      two summed over the query heads that share a KV head (V:124).

    ``out`` (optional, the forward output handed to a backward) switches
    Delta to the FlashAttention-2 convention ``Delta = rowsum(dO * out)``.
    In exact arithmetic ``rowsum(P * dP) = dO . O`` (because ``O = P v``), so
    the two agree for the exact O; with a rounded O they differ by
    ``dO . (out - O)`` per row, and that difference moves dq_r by
    ``-scale * (dO . (out - O)) * sum_j P_rj k_j`` (and dk alike).

    ``delta_terms`` (optional dict) receives, per flattened query row and
    query head, the exact ``Delta`` (``"delta"``, ``[T, Hq]``) and
    ``sum_j P_rj k_j`` (``"pk"``, ``[T, Hq, D]``): the two factors of that
    dq difference, for bounding it.

    A row with no legal key has P = 0 and contributes nothing.  Inputs are CPU
    tensors of the forward's shapes; returns ``(dq, dk, dv)`` in ``dtype``.
    ``rows`` (optional) restricts the work to those flattened query rows: dq
    is then exact on them (0 elsewhere) and dk / dv hold only their share.
    """
    batch, seq_q, hq, d = (int(x) for x in q.shape)
    hkv = int(k.shape[2])
    g = hq // hkv
    scale = (1.0 / d) ** 0.5 if sm_scale is None else float(sm_scale)
    start, end = _bounds_for(q, k, full_idx, local_idx, window_size, metadata)
    qf = q.reshape(batch * seq_q, hq, d).to(dtype)
    kf = k.reshape(-1, hkv, d).to(dtype)
    vf = v.reshape(-1, hkv, d).to(dtype)
    dof = grad_out.reshape(batch * seq_q, hq, d).to(dtype)
    of = None if out is None else out.reshape(batch * seq_q, hq, d).to(dtype)
    if delta_terms is not None:
        delta_terms["delta"] = torch.zeros(batch * seq_q, hq, dtype=dtype)
        delta_terms["pk"] = torch.zeros(batch * seq_q, hq, d, dtype=dtype)
    dq = torch.zeros_like(qf)
    dk = torch.zeros_like(kf)
    dv = torch.zeros_like(vf)
    if rows is None:
        rows = np.concatenate([np.asarray(full_idx, dtype=np.int64).reshape(-1),
                               np.asarray(local_idx, dtype=np.int64).reshape(-1)])
    rows = np.sort(np.asarray(rows, dtype=np.int64))
    for c0 in range(0, rows.size, chunk):
        r = rows[c0:c0 + chunk]
        ks, ke = int(start[r].min()), int(end[r].max())
        if ke <= ks:
            continue
        n = len(r)
        rt = torch.from_numpy(r)
        span = torch.arange(ks, ke)
        legal = (span[None, :] >= torch.from_numpy(start[r])[:, None]) & \
                (span[None, :] < torch.from_numpy(end[r])[:, None])          # [R, L]
        qr = qf[rt].reshape(n, hkv, g, d).permute(1, 0, 2, 3).reshape(hkv, n * g, d)
        dor = dof[rt].reshape(n, hkv, g, d).permute(1, 0, 2, 3).reshape(hkv, n * g, d)
        kc = kf[ks:ke].permute(1, 0, 2).contiguous()                        # [Hkv, L, D]
        vc = vf[ks:ke].permute(1, 0, 2).contiguous()
        s = torch.bmm(qr, kc.transpose(1, 2).contiguous()) * scale          # [Hkv, R*G, L]
        s = s.reshape(hkv, n, g, -1).masked_fill(~legal[None, :, None, :], float("-inf"))
        mx = s.amax(-1, keepdim=True)
        mx = torch.where(torch.isfinite(mx), mx, torch.zeros_like(mx))
        e = torch.exp(s - mx)
        tot = e.sum(-1, keepdim=True)
        p = torch.where(tot > 0, e / torch.where(tot > 0, tot, torch.ones_like(tot)),
                        torch.zeros_like(e)).reshape(hkv, n * g, -1)       # [Hkv, R*G, L]
        dp = torch.bmm(dor, vc.transpose(1, 2).contiguous())                # [Hkv, R*G, L]
        delta = None
        if of is not None:
            # A row with no legal key has O = 0/0 = NaN and P = 0: it contributes
            # nothing, so its Delta is taken as 0.
            orr = of[rt].reshape(n, hkv, g, d).permute(1, 0, 2, 3).reshape(hkv, n * g, d)
            delta = (dor * orr).sum(-1, keepdim=True)
            delta = torch.where((tot > 0).reshape(hkv, n * g, 1), delta, torch.zeros_like(delta))
        ds = _score_grad(p, dp, delta)
        if delta_terms is not None:
            ex = (p * dp).sum(-1)                                           # [Hkv, R*G]
            delta_terms["delta"][rt] = ex.reshape(hkv, n, g).permute(1, 0, 2).reshape(n, hq)
            pk = torch.bmm(p, kc)                                           # [Hkv, R*G, D]
            delta_terms["pk"][rt] = pk.reshape(hkv, n, g, d).permute(1, 0, 2, 3).reshape(n, hq, d)
        dq_r = torch.bmm(ds, kc) * scale                                    # [Hkv, R*G, D]
        dq[rt] = dq_r.reshape(hkv, n, g, d).permute(1, 0, 2, 3).reshape(n, hq, d)
        dk[ks:ke] += (torch.bmm(ds.transpose(1, 2).contiguous(), qr) * scale).permute(1, 0, 2)
        dv[ks:ke] += torch.bmm(p.transpose(1, 2).contiguous(), dor).permute(1, 0, 2)
    return (dq.reshape(batch, seq_q, hq, d), dk.reshape(k.shape[0], -1, hkv, d),
            dv.reshape(v.shape[0], -1, hkv, d))
