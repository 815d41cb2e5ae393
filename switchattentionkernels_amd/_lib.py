"""ctypes binding of ``libswattn.so`` (declared in ``include/swattn.h``).

The library is built in-tree by ``switchattentionkernels_amd.build``.  There
is no fallback: if the library is missing every call raises, so a GPU run can
never silently compute on a different path.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  -- loads PyTorch's HIP runtime before the library

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libswattn.so")

_lock = threading.Lock()
_lib = None

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
    "swattn_decode_workspace_bytes": (ctypes.c_size_t, [_i32, _i64, _i32, _i32]),
    "swattn_decode_fwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i32,
                                         _i32, _i32, _i32, ctypes.c_float, _vp, ctypes.c_size_t,
                                         _vp]),
    "swattn_shard_bounds": (ctypes.c_int, [_vp, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp]),
    "swattn_merge_partials": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i32, _vp,
                                             _vp, _i64, _i32, _vp]),
    "swattn_prefill_fwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp,
                                          _vp, _vp, _i32, _i64, _i64, _i32, _i32, _i32, _i32,
                                          ctypes.c_float, _vp, ctypes.c_size_t, _vp]),
    "swattn_prefill_bwd_workspace_bytes": (ctypes.c_size_t, [_i32, _i64, _i32, _i32, _i32, _i64,
                                                             _i64]),
    "swattn_prefill_bwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _vp,
                                          _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i32, _i32,
                                          _i32, _i32, ctypes.c_float, _vp, ctypes.c_size_t, _vp]),
    "swattn_mfma_peak": (ctypes.c_int, [_i64, _i32, _vp, _vp]),
}


class LibraryNotBuilt(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load (once) and return the library handle with typed entry points."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise LibraryNotBuilt(
                    f"{LIB_PATH} is missing: build it with "
                    "`python -m switchattentionkernels_amd.build`")
            h = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(h, name)
                fn.restype = res
                fn.argtypes = args
            _lib = h
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().swattn_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed with status {status}: {msg}")


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_handle(device) -> int:
    """hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream
