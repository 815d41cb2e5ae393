"""CPU oracle for Switch Attention prefill -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes for the routed
GQA prefill path (YushengZhao/SwitchAttentionKernels, files
``swiattn_gqa_prefill_varlen.py`` = V and ``swiattn_gqa_prefill.py`` = F).
It is the checker for the HIP implementation in ``switchattentionkernels_amd``
and is imported only by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``.  The product path never imports it.

Modules
-------
``routing``   integer work: mask compaction (V:306-322), index checks
              (V:271-304, V:390-393), position metadata (V:27, V:353-383,
              F:145-155).  numpy, bit-exact.
``attention`` floating-point work: dense masked attention in fp32 torch
              (V:103-249) and its backward (the derivative of that
              forward; the reference has none, V:14-15), plus a float64
              pure-Python brute force for tiny inputs used to pin both.

Pinning (how each function is checked, see ``tests/test_oracle.py``)
--------------------------------------------------------------------
* ``compact``              == ``np.flatnonzero`` / ``torch.nonzero``.
* ``check_indices``        fires each reference error on inputs that violate
                           exactly one condition.
* ``default_bounds``       == F's rule, enumerated key by key (F:145-155).
* ``varlen_metadata``      single sequence == ``default_bounds``; packed rows
                           equal per-sequence bounds shifted by the offset.
* ``routed_attention``     == float64 brute force on tiny inputs; p_full=1 ==
                           ``torch.nn.functional.scaled_dot_product_attention``
                           (causal); W >= S == causal; W == 1 gives O = V_i;
                           the routed result is the per-row select of the two
                           dense branches; packed == per-sequence.
* ``routed_flops``         == a direct count of legal (query, key) pairs.
* ``shard_bounds``         whole-sequence chunk == ``default_bounds``; the
                           chunks of any split partition every row's range.
* ``merge_partials``       attention over disjoint key subsets, merged, ==
                           attention over their union (float64 brute force).
* ``decode_attention``     == the last row of ``routed_attention`` run over
                           the cache as a sequence (full and local, W in and
                           out of range, length 1).
* ``routed_attention_backward``
                           == torch autograd through ``routed_attention``;
                           == central finite differences (float64) of the
                           pure-Python brute force, which shares no code with
                           it; sum_j dk_j = 0 and sum_j dv_j = sum_i dO_i per
                           KV head (softmax shift invariance, rows of P sum
                           to one).  With ``out`` (Delta = dO . out, the
                           FlashAttention-2 convention): == the exact
                           gradient for out = O; for a rounded out, dq moves
                           by exactly ``-scale * (dO . (out - O)) * P k`` per
                           row (``delta_shift_bound``), and a dropped or
                           doubled Delta breaks that bound.

Parity of the exact bf16 bits produced by the reference's TileLang kernels is
unpinned (those kernels need TileLang + Hopper, neither exists here); the
contract is the tolerance against this fp32 oracle.
"""

from .routing import (  # noqa: F401
    compact,
    check_indices,
    default_bounds,
    varlen_metadata,
    shard_bounds,
    ERR_FULL_RANGE,
    ERR_FULL_ORDER,
    ERR_LOCAL_RANGE,
    ERR_LOCAL_ORDER,
    ERR_OVERLAP,
)
from .attention import (  # noqa: F401
    routed_attention,
    brute_force_attention,
    routed_flops,
    row_bounds,
    merge_partials,
    decode_attention,
    routed_attention_backward,
    delta_shift_bound,
    LOG2E,
)
