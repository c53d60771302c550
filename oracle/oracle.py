"""CPU oracle for the adaptive hybrid quantization path (TEST INFRASTRUCTURE).

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
bench.py import this module, and only as the checker; the product
(``atlasinfer_amd``) never does.

The arithmetic lives in ``aq_oracle.c`` (built into ``oracle/_build``); this
module wraps it with numpy and restates the reference's storage layout:

* ``quantize``  -> the reference's ``QuantizedTensor`` fields
  (``/root/reference/atlasinfer_core/quant/adaptive_quantizer.py:102-148``):
  ``fp8_data`` = codes of the non-outliers only, block after block, in element
  order (:110,125-126,136); ``fp16_outliers`` and ``outlier_indices`` = values
  and flat indices of the outliers in ascending order (:109-117,137-138);
  ``scale_factors`` = one fp16 per block (:133,139).  The dense code array
  (one byte per padded element, 0 at outliers) is returned too; it is the
  layout the HIP kernels use.
* ``dequantize`` -> ``dequantize_tensor`` (:185-245).
* ``zscore`` -> ``calculate_zscore_manual`` (:44-49).
"""
from __future__ import annotations

import concurrent.futures as cf
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "libaq_oracle.so")
_lib = None

FMT_INT8 = 0
FMT_E4M3 = 1


def build() -> str:
    """Compile aq_oracle.c with the Makefile beside it."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.aqo_h2f.argtypes = [ctypes.c_uint16]
        L.aqo_h2f.restype = ctypes.c_float
        L.aqo_f2h.argtypes = [ctypes.c_float]
        L.aqo_f2h.restype = ctypes.c_uint16
        L.aqo_e4m3_to_double.argtypes = [ctypes.c_uint8]
        L.aqo_e4m3_to_double.restype = ctypes.c_double
        L.aqo_e4m3_encode.argtypes = [ctypes.c_double]
        L.aqo_e4m3_encode.restype = ctypes.c_uint8
        L.aqo_hdiv.argtypes = [ctypes.c_uint16, ctypes.c_uint16]
        L.aqo_hdiv.restype = ctypes.c_uint16
        L.aqo_zscore.argtypes = [P, i64, ctypes.c_float, P, P]
        L.aqo_zscore.restype = None
        L.aqo_quantize.argtypes = [P, i64, i64, ctypes.c_uint16, ctypes.c_int, P, P, P, P]
        L.aqo_quantize.restype = i64
        L.aqo_dequantize.argtypes = [P, P, i64, i64, ctypes.c_int, P, P, i64, P]
        L.aqo_dequantize.restype = None
        L.aqo_init.argtypes = []
        L.aqo_init.restype = None
        L.aqo_init()  # the memoised E4M3 table, before any threaded call
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def threshold_f16(z_threshold: float) -> np.uint16:
    """torch compares an fp16 tensor with a Python float after casting the
    scalar to the tensor dtype (double -> float -> half)."""
    return np.float16(np.float32(z_threshold)).view(np.uint16)


def quantize(w: np.ndarray, block_size: int = 128, z_threshold: float = 3.0, fmt: int = FMT_INT8,
             with_stats: bool = False, threads: int | None = None) -> dict:
    """Quantize fp16 array ``w`` (any shape) as quantize_tensor does.  Large
    inputs are split over up to ``threads`` host threads on block boundaries
    (results identical to one thread)."""
    x = np.ascontiguousarray(w, dtype=np.float16).reshape(-1).view(np.uint16)
    numel = x.size
    G = int(block_size)
    out = {"original_shape": tuple(w.shape), "block_size": G, "fmt": fmt}
    if numel == 0:
        out.update(fp8_data=np.zeros(0, np.int8 if fmt == FMT_INT8 else np.uint8),
                   fp16_outliers=np.zeros(0, np.float16), outlier_indices=np.zeros(0, np.int64),
                   scale_factors=np.zeros(0, np.float16), codes=np.zeros(0, np.uint8),
                   is_outlier=np.zeros(0, np.uint8))
        return out
    nblocks = (numel + G - 1) // G
    padded = nblocks * G
    codes = np.zeros(padded, np.uint8)
    scales = np.zeros(nblocks, np.uint16)
    flags = np.zeros(padded, np.uint8)
    stats = np.zeros(nblocks * 3, np.uint16) if with_stats else None
    L = lib()
    thr = int(threshold_f16(z_threshold))

    def run(b0, b1):
        # blocks [b0, b1): each block is independent, so disjoint block
        # ranges can run in parallel threads (ctypes releases the GIL)
        n = min(numel - b0 * G, (b1 - b0) * G)
        off = lambda a, k: ctypes.c_void_p(a.ctypes.data + k * a.itemsize)  # noqa: E731
        L.aqo_quantize(off(x, b0 * G), n, G, thr, fmt, off(codes, b0 * G), off(scales, b0), off(flags, b0 * G),
                       off(stats, 3 * b0) if stats is not None else None)

    nthreads = max(1, min(threads or (os.cpu_count() or 1), 16, numel // (1 << 18)))
    if nthreads == 1:
        run(0, nblocks)
    else:
        step = -(-nblocks // nthreads)
        with cf.ThreadPoolExecutor(nthreads) as ex:
            list(ex.map(lambda b0: run(b0, min(b0 + step, nblocks)), range(0, nblocks, step)))
    xp = np.zeros(padded, np.uint16)
    xp[:numel] = x
    is_out = flags.astype(bool)
    idx = np.nonzero(is_out)[0].astype(np.int64)
    out.update(
        codes=codes,
        is_outlier=flags,
        scale_factors=scales.view(np.float16),
        outlier_indices=idx,
        fp16_outliers=xp[idx].view(np.float16),
        fp8_data=(codes[~is_out].view(np.int8) if fmt == FMT_INT8 else codes[~is_out]),
    )
    if stats is not None:
        out["stats"] = stats.reshape(nblocks, 3).view(np.float16)
    return out


def dense_codes_from_compact(fp8_data: np.ndarray, outlier_indices: np.ndarray, padded: int) -> np.ndarray:
    """Undo the reference's compaction: put the non-outlier codes back at
    their element positions (0 at outliers)."""
    dense = np.zeros(padded, np.uint8)
    mask = np.ones(padded, bool)
    mask[outlier_indices] = False
    dense[mask] = fp8_data.view(np.uint8)
    return dense


def dequantize(q: dict) -> np.ndarray:
    """dequantize_tensor: fp16 array of q['original_shape']."""
    shape = q["original_shape"]
    numel = int(np.prod(shape)) if len(shape) else 1
    if numel == 0:
        return np.zeros(shape, np.float16)
    G = q["block_size"]
    padded = (numel + G - 1) // G * G
    codes = q.get("codes")
    if codes is None:
        codes = dense_codes_from_compact(q["fp8_data"], q["outlier_indices"], padded)
    out = np.zeros(numel, np.uint16)
    idx = np.ascontiguousarray(q["outlier_indices"], np.int64)
    vals = np.ascontiguousarray(q["fp16_outliers"], np.float16).view(np.uint16)
    scales = np.ascontiguousarray(q["scale_factors"], np.float16).view(np.uint16)
    lib().aqo_dequantize(_ptr(np.ascontiguousarray(codes, np.uint8)), _ptr(scales), numel, G, q["fmt"],
                         _ptr(idx), _ptr(vals), idx.size, _ptr(out))
    return out.view(np.float16).reshape(shape)


def zscore(x: np.ndarray, eps: float = 1e-6):
    """calculate_zscore_manual for a 1-D fp16 array; returns (z, (mean, std, den))."""
    a = np.ascontiguousarray(x, np.float16).reshape(-1).view(np.uint16)
    z = np.zeros(a.size, np.uint16)
    st = np.zeros(3, np.uint16)
    lib().aqo_zscore(_ptr(a), a.size, float(np.float32(eps)), _ptr(z), _ptr(st))
    return z.view(np.float16), tuple(st.view(np.float16))


def e4m3_encode_all_f16() -> np.ndarray:
    """E4M3 code of clamp(v, +-448) for every fp16 bit pattern v (0..65535)."""
    L = lib()
    out = np.zeros(65536, np.uint8)
    for b in range(65536):
        v = L.aqo_h2f(b)
        if v == v:
            v = min(max(v, -448.0), 448.0)
        out[b] = L.aqo_e4m3_encode(v)
    return out


def qlinear_reference(x: np.ndarray, w_deq: np.ndarray, bias=None) -> np.ndarray:
    """F.linear(x, W, b) in float64 from fp16 operands (the tolerance
    reference for the fused kernels; atlas_wrappers.py:67)."""
    y = x.astype(np.float64) @ w_deq.astype(np.float64).T
    if bias is not None:
        y = y + bias.astype(np.float64)
    return y
