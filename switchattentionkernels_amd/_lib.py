"""ctypes binding of ``libswattn.so`` (declared in ``include/swattn.h``).

The library is built in-tree by ``switchattentionkernels_amd.build``.  There
is no fallback: if the library is missing every call raises, so a GPU run can
never silently compute on a different path.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading

import torch  # noqa: F401  -- loads PyTorch's HIP runtime before the library

from ._abi import PROBE_SIGNATURES, SIGNATURES, bind  # noqa: F401  -- part of this module's API

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libswattn.so")
PROBE_PATH = os.path.join(_HERE, "libswattn_probe.so")

_lock = threading.Lock()
_lib = None
_probe = None


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
            _lib = bind(ctypes.CDLL(LIB_PATH))
    return _lib


def probe_lib() -> ctypes.CDLL:
    """bench.py's measurement probe (``libswattn_probe.so``), loaded once."""
    global _probe
    with _lock:
        if _probe is None:
            if not os.path.exists(PROBE_PATH):
                raise LibraryNotBuilt(f"{PROBE_PATH} is missing: build it with "
                                      "`python -m switchattentionkernels_amd.build`")
            _probe = bind(ctypes.CDLL(PROBE_PATH), PROBE_SIGNATURES)
    return _probe


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().swattn_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed with status {status}: {msg}")


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_no_switch = contextlib.nullcontext()


def _index(device) -> int:
    idx = device.index
    return torch.cuda.current_device() if idx is None else idx


def stream_handle(device) -> int:
    """hipStream_t of torch's current stream on ``device``."""
    if _raw_stream is not None:
        return _raw_stream(_index(device))
    return torch.cuda.current_stream(device).cuda_stream


def on_device(device):
    """``torch.cuda.device(device)``, or a context that does nothing when
    ``device`` is already the current device (the common case, and a
    tenth of the cost)."""
    idx = device.index
    if idx is None or idx == torch.cuda.current_device():
        return _no_switch
    return torch.cuda.device(idx)
