"""MI355X-native Switch Attention GQA prefill.

Drop-in for the Python API of YushengZhao/SwitchAttentionKernels
(``swiattn_gqa_prefill_varlen.py``): routed prefill where every query token is
hard-routed to full causal attention or causal sliding-window attention.
Device work runs in hand-written gfx950 HIP kernels behind the C ABI of
``libswattn.so`` (``include/swattn.h``).
"""

from .prefill import (  # noqa: F401
    build_switch_query_indices,
    build_switch_query_indices_from_logits,
    switch_gqa_prefill_forward,
    switch_gqa_prefill_varlen_forward,
)
from .metadata import SwitchAttentionMetadata, build_switch_attention_metadata  # noqa: F401
from .flops import routed_flops  # noqa: F401
from .split import merge_attention_partials, shard_attention_metadata  # noqa: F401
from .decode import switch_gqa_decode_forward  # noqa: F401
from .backward import (  # noqa: F401
    SwitchGQAPrefillFunction,
    switch_gqa_prefill,
    switch_gqa_prefill_backward,
    switch_gqa_prefill_varlen,
)

__all__ = [
    "build_switch_query_indices",
    "build_switch_query_indices_from_logits",
    "switch_gqa_prefill_forward",
    "switch_gqa_prefill_varlen_forward",
    "SwitchAttentionMetadata",
    "build_switch_attention_metadata",
    "routed_flops",
    "shard_attention_metadata",
    "merge_attention_partials",
    "switch_gqa_decode_forward",
    "switch_gqa_prefill_backward",
    "switch_gqa_prefill",
    "switch_gqa_prefill_varlen",
    "SwitchGQAPrefillFunction",
]
