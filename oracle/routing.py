"""Integer side of the Switch Attention oracle (numpy, bit-exact).

TEST INFRASTRUCTURE ONLY -- see the package docstring.  Reference file tags:
V = swiattn_gqa_prefill_varlen.py, F = swiattn_gqa_prefill.py.
"""

from __future__ import annotations

import numpy as np

# Error bits, in the order the reference raises them (V:384-393).
ERR_FULL_RANGE = 1    # V:299-300 on the full list
ERR_FULL_ORDER = 2    # V:301-302 on the full list
ERR_LOCAL_RANGE = 4   # V:299-300 on the local list
ERR_LOCAL_ORDER = 8   # V:301-302 on the local list
ERR_OVERLAP = 16      # documented contract (V:341-342, README:81); not checked by V

MSG_RANGE = "query index is outside [0, sequence_length)"          # V:300
MSG_ORDER = "query indices must be strictly increasing"           # V:302
MSG_COVER = "full and local query lists must cover the sequence"  # V:393
MSG_DISJOINT = "full and local query lists must be disjoint"


def compact(mask) -> tuple[np.ndarray, np.ndarray]:
    """Stream-compact a hard route mask into (full, local) ascending int32 lists.

    Restates ``build_switch_query_indices`` (V:306-322): the reference returns
    ``arange(S)[mask]`` and ``arange(S)[~mask]``.  Here it is written as the
    exclusive-prefix-sum scatter that the GPU kernel implements: element i goes
    to slot ``excl(i)`` of the full list when routed full and to slot
    ``i - excl(i)`` of the local list otherwise, where ``excl(i)`` counts the
    full-routed elements before i.  A ``[B, S]`` mask is flattened row-major,
    so positions are ``b * S + i``.
    """
    m = np.asarray(mask).reshape(-1).astype(bool)
    n = m.size
    pos = np.arange(n, dtype=np.int64)
    mi = m.astype(np.int64)
    excl = np.cumsum(mi) - mi
    n_full = int(mi.sum())
    full = np.empty(n_full, dtype=np.int32)
    local = np.empty(n - n_full, dtype=np.int32)
    full[excl[m]] = pos[m]
    local[(pos - excl)[~m]] = pos[~m]
    return full, local


def check_indices(full, local, seq_len: int) -> int:
    """Return the error bits the reference's index checks would raise on.

    Restates the device-side checks of ``_prepare_indices`` (V:299-302) for each
    list.  ``ERR_OVERLAP`` covers the documented "disjoint" precondition
    (V:341-342); it can only fire when both lists are valid and their lengths
    sum to ``seq_len`` (then overlap <=> a missing position).
    """
    flags = 0
    f = np.asarray(full, dtype=np.int64).reshape(-1)
    l = np.asarray(local, dtype=np.int64).reshape(-1)
    if f.size and ((f < 0) | (f >= seq_len)).any():
        flags |= ERR_FULL_RANGE
    if f.size > 1 and (f[1:] <= f[:-1]).any():
        flags |= ERR_FULL_ORDER
    if l.size and ((l < 0) | (l >= seq_len)).any():
        flags |= ERR_LOCAL_RANGE
    if l.size > 1 and (l[1:] <= l[:-1]).any():
        flags |= ERR_LOCAL_ORDER
    if f.size and l.size and np.intersect1d(f, l).size:
        flags |= ERR_OVERLAP
    return flags


def first_error(full, local, seq_len: int):
    """(exception type, message) the reference raises first, or None.

    Order follows V:384-393: full list range, full list order, local list range,
    local list order, coverage by count; the disjointness check runs last.
    """
    flags = check_indices(full, local, seq_len)
    n = np.asarray(full).size + np.asarray(local).size
    if flags & ERR_FULL_RANGE:
        return ValueError, MSG_RANGE
    if flags & ERR_FULL_ORDER:
        return ValueError, MSG_ORDER
    if flags & ERR_LOCAL_RANGE:
        return ValueError, MSG_RANGE
    if flags & ERR_LOCAL_ORDER:
        return ValueError, MSG_ORDER
    if n != seq_len:
        return ValueError, MSG_COVER
    if flags & ERR_OVERLAP:
        return ValueError, MSG_DISJOINT
    return None


def default_bounds(batch: int, seq_q: int, seq_kv: int, window: int):
    """Per-row key bounds without metadata, over flattened rows ``b*Sq + i``.

    F's rule (F:145-155): a query at position i of batch b may attend key j of
    the same batch iff ``j <= i`` and ``j < Skv``; the local branch also needs
    ``j >= max(i - W + 1, 0)``.  Returned in flattened key coordinates
    ``b*Skv + j`` as half-open ``[start, end)`` arrays (full_starts,
    local_starts, ends), each int64 of length ``batch * seq_q``.
    """
    rows = np.arange(batch * seq_q, dtype=np.int64)
    b = rows // seq_q
    i = rows - b * seq_q
    base = b * seq_kv
    ends = base + np.minimum(i + 1, seq_kv)
    full_starts = base.copy()
    local_starts = base + np.maximum(i - window + 1, 0)
    return full_starts, local_starts, ends


def varlen_metadata(cu_seqlens_q, cu_seqlens_kv, window: int) -> dict:
    """Position metadata for packed sequences (the module V imports at V:27).

    V never ships ``build_switch_attention_metadata``; its kernel reads
    ``FullStarts/LocalStarts/CausalEnds`` per query row (V:134-137,
    V:186-193), and the wrapper checks seven int32 vectors (V:360-383).  The
    restatement applies F's rule inside every segment: for query i of segment
    s (0-based inside it) with KV segment ``[ks, ke)``:
    ``full_starts = ks``, ``local_starts = ks + max(i - W + 1, 0)``,
    ``causal_ends = ks + min(i + 1, ke - ks)``.  ``*_positions`` are the
    0-based positions inside the segment and ``*_segment_ids`` the segment
    index.  (The exact contents of the absent module are parity-unpinned.)
    """
    cq = np.asarray(cu_seqlens_q, dtype=np.int64)
    ck = np.asarray(cu_seqlens_kv, dtype=np.int64)
    tq, tk = int(cq[-1]), int(ck[-1])
    out = {k: np.zeros(n, dtype=np.int32) for k, n in (
        ("q_positions", tq), ("kv_positions", tk), ("q_segment_ids", tq),
        ("kv_segment_ids", tk), ("full_starts", tq), ("local_starts", tq),
        ("causal_ends", tq))}
    for s in range(cq.size - 1):
        q0, q1, k0, k1 = int(cq[s]), int(cq[s + 1]), int(ck[s]), int(ck[s + 1])
        i = np.arange(q1 - q0, dtype=np.int64)
        out["q_positions"][q0:q1] = i
        out["q_segment_ids"][q0:q1] = s
        out["full_starts"][q0:q1] = k0
        out["local_starts"][q0:q1] = k0 + np.maximum(i - window + 1, 0)
        out["causal_ends"][q0:q1] = k0 + np.minimum(i + 1, k1 - k0)
        out["kv_positions"][k0:k1] = np.arange(k1 - k0)
        out["kv_segment_ids"][k0:k1] = s
    return out


def shard_bounds(q_positions, kv_start: int, kv_end: int, window: int):
    """Key bounds of query rows at global positions against the key chunk
    ``[kv_start, kv_end)`` of one causal sequence, in chunk coordinates.

    Global legal keys are F's rule (F:145-155): ``[0, p]`` for the full branch
    and ``[max(p - W + 1, 0), p]`` for the local branch.  Each range is cut to
    the chunk and shifted by ``-kv_start``; an empty cut is ``start == end``.
    Returns (full_starts, local_starts, ends) as int64 arrays.
    """
    p = np.asarray(q_positions, dtype=np.int64)
    n = kv_end - kv_start

    def clip(g):
        return np.clip(g - kv_start, 0, n)

    ends = clip(p + 1)
    full_starts = np.minimum(clip(np.zeros_like(p)), ends)
    local_starts = np.minimum(clip(p - window + 1), ends)
    return full_starts, local_starts, ends
