"""Typed signatures of the C ABI declared in ``include/swattn.h``.

Pure ctypes, no torch: the host-side sanitizer test loads the library with
these signatures in a process that does not import torch.
"""

from __future__ import annotations

import ctypes

_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

# name -> (restype, argtypes); must mirror include/swattn.h exactly.
SIGNATURES = {
    "swattn_version": (ctypes.c_int, []),
    "swattn_last_error": (ctypes.c_char_p, []),
    "swattn_compact_workspace_bytes": (ctypes.c_size_t, [_i64]),
    "swattn_compact": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "swattn_compact_logits": (ctypes.c_int, [_vp, _i32, _i64, ctypes.c_float, _vp, _vp, _vp,
                                             ctypes.c_size_t, _vp]),
    "swattn_check_indices": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _vp, _vp]),
    "swattn_build_metadata": (ctypes.c_int, [_vp, _vp, _i32, _i64, _i64, _i32,
                                             _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "swattn_prefill_workspace_bytes": (ctypes.c_size_t, [_i32, _i64, _i32, _i32]),
    "swattn_prefill_split_workspace_bytes": (ctypes.c_size_t, [_i32, _i64, _i64, _i32, _i32,
                                                               _i32, _i32, _i64, _i64]),
    "swattn_decode_workspace_bytes": (ctypes.c_size_t, [_i32, _i64, _i32, _i32]),
    "swattn_decode_fwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i32,
                                         _i32, _i32, _i32, ctypes.c_float, _vp, ctypes.c_size_t,
                                         _vp]),
    "swattn_decode_fwd_noalloc": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64,
                                                 _i32, _i32, _i32, _i32, ctypes.c_float, _vp]),
    "swattn_shard_bounds": (ctypes.c_int, [_vp, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp]),
    "swattn_merge_partials": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i32, _vp,
                                             _vp, _i64, _i32, _vp]),
    "swattn_prefill_fwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp,
                                          _vp, _vp, _i32, _i64, _i64, _i32, _i32, _i32, _i32,
                                          ctypes.c_float, _vp, ctypes.c_size_t, _vp]),
    "swattn_prefill_bwd_workspace_bytes": (ctypes.c_size_t, [_i32, _i64, _i32, _i32, _i32, _i32,
                                                             _i64, _i64]),
    "swattn_prefill_bwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _vp,
                                          _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i32, _i32,
                                          _i32, _i32, ctypes.c_float, _vp, ctypes.c_size_t, _vp]),
}

# libswattn_probe.so (bench.py's measurement probe; not part of swattn.h).
PROBE_SIGNATURES = {
    "swattn_mfma_peak": (ctypes.c_int, [_i64, _i32, _vp, _vp]),
}


def bind(handle: ctypes.CDLL, signatures=None) -> ctypes.CDLL:
    """Set restype / argtypes of every entry point on a loaded library."""
    for name, (res, args) in (SIGNATURES if signatures is None else signatures).items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    return handle
