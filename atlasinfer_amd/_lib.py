"""ctypes binding of libatlasinfer_amd.so (declared in include/atlasinfer_amd.h).

torch is imported first on purpose: the library's HIP runtime dependency
(libamdhip64.so.7) then resolves to the runtime torch already loaded, so
device pointers and streams from torch are valid inside the library.

There is no fallback: if the library is missing or no HIP device is present,
every compute entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libatlasinfer_amd.so")
ABI_VERSION = 10

FMT_INT8 = 0
FMT_E4M3 = 1
FORMATS = {"int8": FMT_INT8, "e4m3": FMT_E4M3}
LAYOUT_FLAT = 0
LAYOUT_TILED = 1
LAYOUTS = {"flat": LAYOUT_FLAT, "tiled": LAYOUT_TILED}
MAX_GROUP = 4

# every function the header declares: name -> (restype, argtypes)
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32P = ctypes.c_void_p
SIGNATURES = {
    "aq_abi_version": (ctypes.c_int, []),
    "aq_last_error": (ctypes.c_char_p, []),
    "aq_max_block_size": (_I64, []),
    "aq_quantize_workspace_size": (_I64, [_I64, _I64]),
    "aq_quantize": (ctypes.c_int, [_P, _I64, _I64, ctypes.c_uint16, ctypes.c_int, _I64, ctypes.c_int, _P, _P, _I32P,
                                   _P, _I64, _P]),
    "aq_quantize_grouped": (ctypes.c_int, [_I64, _P, _P, _I64, ctypes.c_uint16, ctypes.c_int, _I64, ctypes.c_int, _P,
                                           _P, _P, _P, _P, _I32P, _P]),
    "aq_quantize_finish": (ctypes.c_int, [_I64, _I64, _I64, _I32P, _I64, _P, _I64, _P, _P, _I32P, _P]),
    "aq_segment_offsets": (ctypes.c_int, [_P, _I64, _I64, _I64, _I32P, _P]),
    "aq_outlier_cols": (ctypes.c_int, [_P, _I64, _I64, _I32P, _P]),
    "aq_outlier_tiles": (ctypes.c_int, [_I32P, _I32P, _P, _I64, _I64, _I32P, _P, _I32P, _P]),
    "aq_quantize_finish_tiles": (ctypes.c_int, [_I64, _I64, _I64, _I32P, _I64, _P, _I64, _P, _P, _I32P, _I32P, _P,
                                                _I32P, _P]),
    "aq_quantize_finish_tiles_grouped": (ctypes.c_int, [_I64, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                                        _I32P, _P]),
    "aq_compact_codes": (ctypes.c_int, [_P, _I64, _P, _I64, _P, _P]),
    "aq_expand_codes": (ctypes.c_int, [_P, _I64, _P, _I64, _P, _P]),
    "aq_tile_codes": (ctypes.c_int, [_P, _I64, _I64, _P, _P]),
    "aq_untile_codes": (ctypes.c_int, [_P, _I64, _I64, _P, _P]),
    "aq_dequantize": (ctypes.c_int, [_P, _P, _I64, _I64, ctypes.c_int, _I64, ctypes.c_int, _P, _P, _I64, _P, _P]),
    "aq_zscore": (ctypes.c_int, [_P, _I64, ctypes.c_float, _P, _P, _P]),
    "aq_qlinear_workspace_size": (_I64, [_I64, _I64, _I64]),
    "aq_qlinear": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _P, _I64, ctypes.c_int, _I32P, _I32P, _P, _I32P, _P,
                                  _I64, _P, _P, _P, _I64, _P]),
    "aq_qlinear_grouped": (ctypes.c_int, [_P, _I64, _I64, ctypes.c_int, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                          _P, _P, _P, _P, _I64, _P]),
    "aq_qlinear_noalloc": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _P, _I64, ctypes.c_int, _I32P, _I32P, _P,
                                          _I32P, _P, _I64, _P, _P, _P]),
    "aq_decode_attention": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, ctypes.c_float,
                                           ctypes.c_float, _P, _P, _P, _I64, _P, _P]),
    "aq_qlinear_decode": (ctypes.c_int, [_P, _I64, _I64, ctypes.c_int, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                         _P, _P, ctypes.c_int,
                                         _P, _P, _P, ctypes.c_float, _P, _P, _P]),
    "aq_decode_norm": (ctypes.c_int, [_P, _P, _P, _P, ctypes.c_float, _I64, _I64, ctypes.c_int, _P, _P]),
    "aq_silu_mul": (ctypes.c_int, [_P, _P, _P, _I64, _P]),
    "aq_decode_attention_workspace": (ctypes.c_int64, [_I64, _I64, _I64, _I64, _I64]),
}
NOALLOC_SCRATCH_BYTES = 64 << 20  # AQ_NOALLOC_SCRATCH_BYTES


def ptr_array(values, ctype=ctypes.c_void_p):
    """A host array of pointers / ints for the grouped entry points."""
    return (ctype * len(values))(*values)


_lib = None
_lock = threading.Lock()


class AQError(RuntimeError):
    """A call into libatlasinfer_amd failed (message from aq_last_error())."""


def load() -> ctypes.CDLL:
    """Load the library once; raise if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise AQError(f"{LIB_PATH} is missing: build it with `python -m atlasinfer_amd.build` "
                              "(the MI355X path has no CPU fallback)")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                f = getattr(L, name)
                f.restype = res
                f.argtypes = args
            v = L.aq_abi_version()
            if v != ABI_VERSION:
                raise AQError(f"libatlasinfer_amd ABI version {v}, expected {ABI_VERSION}")
            _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().aq_last_error().decode(errors="replace")
        raise AQError(f"{what} failed (status {rc}): {msg}")


def ptr(t) -> int | None:
    """Device address of a tensor (None for None / empty tensors)."""
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """The handle of torch's current stream on ``device`` (the raw query when
    torch has it: a tenth of the cost of building a Stream object, which
    matters on the per-token decode path)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def compute_device(preferred: torch.device | None = None) -> torch.device:
    """The HIP device the kernels run on: the tensor's own if it lives on one,
    else the current one.  Raises when there is none."""
    if preferred is not None and preferred.type == "cuda":
        return preferred
    if not torch.cuda.is_available():
        raise AQError("atlasinfer_amd needs a HIP (MI355X) device; none is visible")
    return torch.device("cuda", torch.cuda.current_device())
