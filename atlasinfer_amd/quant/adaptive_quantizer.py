"""Adaptive hybrid FP8/FP16 weight quantization on MI355X (gfx950).

Same API as the reference module
/root/reference/atlasinfer_core/quant/adaptive_quantizer.py (also importable
under that name, ``atlasinfer_core.quant.adaptive_quantizer``):

* ``QuantizedTensor``          (reference :8-42) -- the six reference fields in
  order, plus trailing fields with defaults: ``code_format``,
  ``outlier_row_ptr`` (CSR row pointer, int32 [N+1]), ``outlier_cols``
  (int32 [nnz]), ``code_layout``, and the same outliers listed per block of
  16 rows x 64 columns for the dequant-GEMM (``outlier_tile_ptr``,
  ``outlier_tile_ent``, see ``aq_outlier_tiles`` in include/atlasinfer_amd.h).
* ``calculate_zscore_manual``  (reference :44-49)
* ``quantize_tensor``          (reference :51-148)
* ``dequantize_tensor``        (reference :156-251)
* ``clear_dequantized_cache``  (reference :253-263)

Every computation runs in the HIP kernels of libatlasinfer_amd.so; CPU inputs
are copied to the GPU, processed there and the results copied back to the
input's device.  Without a HIP device the compute functions raise.

Code formats:
* ``"int8"`` -- the reference's format, bit for bit: ``fp8_data`` holds the
  int8 codes of the non-outliers only, in element order.
* ``"e4m3"`` (default) -- OCP FP8 E4M3 codes computed by the same op
  sequence with 448 in place of 127; ``fp8_data`` is the dense code array
  (torch.float8_e4m3fn, one code per element, 0 at outliers).  For weights
  whose rows tile (2-D view [N, K] with N % 16 == 0, K % 128 == 0, blocks of
  a multiple of 32 dividing K) the codes are stored in the tiled layout the
  quantized-linear kernels read (``code_layout == "tiled"``: 16 x 128 tiles,
  see include/atlasinfer_amd.h); ``dense_codes()`` returns element order.
``block_size=-1`` selects one block per output channel (block = last dim).
"""
from __future__ import annotations

import ctypes
import threading
from typing import NamedTuple, Optional

import numpy as np
import torch

from .. import _lib

DEFAULT_CODE_FORMAT = "e4m3"
PER_CHANNEL = -1


class DeviceInt:
    """An int that still lives in a one-element device tensor: read (one host
    sync) the first time it is used as a number -- converted, compared,
    tested for truth, hashed or used in arithmetic -- then kept.  Lets
    quantize_tensor hand back the largest block-list count without waiting
    for it; the first consumer (the GEMM's kernel choice, serialization)
    pays the wait.  That first use makes a device-to-host copy, which HIP
    graph capture does not allow: a caller that captures should use the
    value once before capturing (GraphDecoder's eager warm-up steps do)."""
    __slots__ = ("_t", "_i", "_v")

    def __init__(self, t: torch.Tensor, index: Optional[int] = None):
        # the value is t[index] (t itself when index is None)
        self._t, self._i, self._v = t, index, None

    def _get(self) -> int:
        if self._v is None:
            self._v = int((self._t if self._i is None else self._t[self._i]).item())
            self._t = None
        return self._v

    def __int__(self):
        return self._get()

    __index__ = __int__

    def __eq__(self, o):
        return self._get() == int(o)

    def __lt__(self, o):
        return self._get() < int(o)

    def __le__(self, o):
        return self._get() <= int(o)

    def __gt__(self, o):
        return self._get() > int(o)

    def __ge__(self, o):
        return self._get() >= int(o)

    def __ne__(self, o):
        return self._get() != int(o)

    def __bool__(self):
        return self._get() != 0

    def __hash__(self):
        return hash(self._get())

    def __mul__(self, o):
        return self._get() * o

    __rmul__ = __mul__

    def __add__(self, o):
        return self._get() + o

    __radd__ = __add__

    def __sub__(self, o):
        return self._get() - o

    def __repr__(self):
        return repr(self._get())


class QuantizedTensor(NamedTuple):
    """A tensor quantized into the hybrid FP8/FP16 format (reference :8-18)."""
    fp8_data: torch.Tensor          # codes (int8 compacted stream, or dense e4m3)
    fp16_outliers: torch.Tensor     # fp16 outlier values, ascending flat index order
    outlier_indices: torch.Tensor   # int64 flat indices of the outliers (padded tensor)
    scale_factors: torch.Tensor     # fp16, one per block
    original_shape: torch.Size
    block_size: int
    code_format: str = "int8"
    outlier_row_ptr: Optional[torch.Tensor] = None  # int32 [N + 1] over the last dim
    outlier_cols: Optional[torch.Tensor] = None     # int32 [nnz]
    code_layout: str = "flat"                       # "flat" (element order) or "tiled"
    outlier_tile_ptr: Optional[torch.Tensor] = None  # int32 [(N/16)*(K/64) + 1]
    outlier_tile_ent: Optional[torch.Tensor] = None  # int32 [nnz + 64], packed entries
    outlier_tile_max: int = 0                        # most entries in one block (an int or a DeviceInt)

    def to(self, device):
        """Move every tensor to ``device``; returns self when already there
        (reference :20-32)."""
        device = torch.device(device)
        if self.fp8_data.device == device:
            return self
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        return self._replace(
            fp8_data=mv(self.fp8_data),
            fp16_outliers=mv(self.fp16_outliers),
            outlier_indices=mv(self.outlier_indices),
            scale_factors=mv(self.scale_factors),
            outlier_row_ptr=mv(self.outlier_row_ptr),
            outlier_cols=mv(self.outlier_cols),
            outlier_tile_ptr=mv(self.outlier_tile_ptr),
            outlier_tile_ent=mv(self.outlier_tile_ent),
        )

    def memory_footprint(self, include_overhead=True) -> int:
        """Bytes held by the component tensors (+128 when include_overhead,
        reference :34-42)."""
        mem = 0
        for t in (self.fp8_data, self.fp16_outliers, self.outlier_indices, self.scale_factors,
                  self.outlier_row_ptr, self.outlier_cols, self.outlier_tile_ptr, self.outlier_tile_ent):
            if t is not None:
                mem += t.element_size() * t.nelement()
        if include_overhead:
            mem += 128
        return mem


def _format_id(code_format: str) -> int:
    try:
        return _lib.FORMATS[code_format]
    except KeyError:
        raise ValueError(f"code_format must be one of {sorted(_lib.FORMATS)}, got {code_format!r}") from None


def _threshold_bits(z_threshold: float) -> int:
    # torch compares an fp16 tensor with a Python float after casting the
    # scalar to fp16 (double -> float -> half)
    return int(np.float16(np.float32(z_threshold)).view(np.uint16))


def _resolve_block(block_size: int, shape: torch.Size) -> int:
    if block_size == PER_CHANNEL:
        return int(shape[-1]) if len(shape) >= 1 and shape[-1] > 0 else 1
    if not isinstance(block_size, (int, np.integer)) or block_size < 1:
        raise ValueError(f"block_size must be a positive int or -1 (per output channel), got {block_size!r}")
    return int(block_size)


def calculate_zscore_manual(data: torch.Tensor, eps=1e-6) -> torch.Tensor:
    """(data - mean) / (std + eps) over all of ``data`` with fp16 tensor
    semantics (reference :44-49).  fp16 only; at most 65536 elements."""
    if data.dtype != torch.float16:
        raise TypeError(f"calculate_zscore_manual: float16 input expected, got {data.dtype}")
    L = _lib.load()
    n = data.numel()
    if n == 0:
        return torch.empty_like(data)
    if n > L.aq_max_block_size():
        raise ValueError(f"calculate_zscore_manual: {n} elements exceed the {L.aq_max_block_size()} limit")
    dev = _lib.compute_device(data.device)
    x = data.to(dev).contiguous().view(-1)
    z = torch.empty_like(x)
    _lib.check(L.aq_zscore(_lib.ptr(x), n, float(eps), _lib.ptr(z), None, _lib.stream_of(dev)), "aq_zscore")
    return z.view(data.shape).to(data.device)


def _rows_cols(shape) -> tuple:
    K = int(shape[-1]) if len(shape) >= 1 else 1
    numel = 1
    for d in shape:
        numel *= int(d)
    return (numel // K if K else 0), K


def tiled_eligible(shape, block_size: int) -> bool:
    """Whether codes of a weight of this shape can use the tiled layout (and
    the fused quantized-linear kernels)."""
    if len(shape) < 2:
        return False
    N, K = _rows_cols(shape)
    G = block_size
    return N > 0 and N % 16 == 0 and K >= 128 and K % 128 == 0 and G >= 32 and G % 32 == 0 and K % G == 0


def _empty(original_shape, block_size, fmt_name, device) -> QuantizedTensor:
    code_dtype = torch.int8 if fmt_name == "int8" else torch.float8_e4m3fn
    n = int(original_shape[0]) if len(original_shape) >= 2 else 1
    return QuantizedTensor(
        fp8_data=torch.empty((0,), dtype=code_dtype, device=device),
        fp16_outliers=torch.empty((0,), dtype=torch.float16, device=device),
        outlier_indices=torch.empty((0,), dtype=torch.long, device=device),
        scale_factors=torch.empty((0,), dtype=torch.float16, device=device),
        original_shape=original_shape,
        block_size=block_size,
        code_format=fmt_name,
        outlier_row_ptr=torch.zeros((max(n, 0) + 1 if len(original_shape) >= 2 else 1,), dtype=torch.int32,
                                    device=device),
        outlier_cols=torch.empty((0,), dtype=torch.int32, device=device),
    )


def quantize_tensor(
    fp16_tensor: torch.Tensor,
    block_size: int = 128,
    z_threshold: float = 3.0,
    *,
    code_format: str = DEFAULT_CODE_FORMAT,
) -> QuantizedTensor:
    """Quantize an fp16 tensor into the hybrid format (reference :51-148).

    Per block of ``block_size`` elements of the flattened, zero-padded tensor:
    elements with |z| > z_threshold are kept as fp16 outliers, the rest are
    coded against one fp16 scale per block.  Results land on the input's
    device.
    """
    if not isinstance(fp16_tensor, torch.Tensor):
        raise TypeError(f"Input must be a PyTorch Tensor, got {type(fp16_tensor)}")
    if fp16_tensor.dtype != torch.float16:
        print(f"Warning: Input tensor was {fp16_tensor.dtype}, converting to FP16 for quantization.")
        fp16_tensor = fp16_tensor.to(torch.float16)
    fmt = _format_id(code_format)
    input_device = fp16_tensor.device
    original_shape = fp16_tensor.shape
    numel = fp16_tensor.numel()
    G = _resolve_block(block_size, original_shape)
    if numel == 0:
        return _empty(original_shape, G, code_format, input_device)

    p = _quantize_prepare(fp16_tensor, G, z_threshold, code_format, fmt)
    L = _lib.load()
    _lib.check(L.aq_quantize(*p["args"], p["stream"]), "aq_quantize")
    nnz = int(p["block_off"][p["nblocks"]].item())  # the one host sync: sizes the outlier tensors
    return _quantize_complete(p, nnz)


def _member_prepare(fp16_tensor: torch.Tensor, G: int, fmt: int, code_format: str, layout: str,
                    dev: torch.device) -> dict:
    """The outputs of one tensor's quantize (numel > 0, fp16) that do not
    depend on its outlier count: codes (E4M3 codes allocated as
    float8_e4m3fn, the dtype they are handed out in; int8 codes as bytes in
    element order, compacted later), scales, block offsets and, for the
    tiled layout, the block lists' pointer array."""
    original_shape = fp16_tensor.shape
    numel = fp16_tensor.numel()
    x = fp16_tensor if fp16_tensor.device == dev and fp16_tensor.is_contiguous() else \
        fp16_tensor.to(dev).contiguous()
    N, K = _rows_cols(original_shape)
    nblocks = (numel + G - 1) // G
    padded = nblocks * G
    codes = torch.empty(padded, dtype=torch.float8_e4m3fn if fmt == _lib.FMT_E4M3 else torch.uint8, device=dev)
    scales = torch.empty(nblocks, dtype=torch.float16, device=dev)
    block_off = torch.empty(nblocks + 1, dtype=torch.int32, device=dev)
    tile_ptr = None
    if layout == "tiled":
        tile_ptr = torch.empty((N // 16) * (K // 64) + 1, dtype=torch.int32, device=dev)
    return dict(x=x, input_device=fp16_tensor.device, original_shape=original_shape, numel=numel, G=G, N=N, K=K,
                nblocks=nblocks, padded=padded, layout=layout, codes=codes, scales=scales, block_off=block_off,
                tile_ptr=tile_ptr, fmt=fmt, code_format=code_format, dev=dev)


def _a256(n: int) -> int:
    return (n + 255) // 256 * 256


def _run_plan(tensors, G: int, fmt: int, code_format: str, dev: torch.device):
    """The members of a tiled run before anything is allocated for them, and
    the byte offsets of their codes, scales, block offsets and block-list
    pointers in one buffer for the run (each 256-byte aligned)."""
    ps, at = [], 0
    for t in tensors:
        numel = t.numel()
        x = t if t.device == dev and t.is_contiguous() else t.to(dev).contiguous()
        N, K = _rows_cols(t.shape)
        nblocks = (numel + G - 1) // G
        ntile = (N // 16) * (K // 64) + 1
        p = dict(x=x, input_device=t.device, original_shape=t.shape, numel=numel, G=G, N=N, K=K, nblocks=nblocks,
                 padded=nblocks * G, ntile=ntile, layout="tiled", fmt=fmt, code_format=code_format, dev=dev)
        offs = []
        for nb in (nblocks * G, 2 * nblocks, 4 * (nblocks + 1), 4 * ntile):  # codes, scales, offsets, pointers
            offs.append(at)
            at += _a256(nb)
        p["at"] = tuple(offs)
        ps.append(p)
    return ps, at


def _run_views(ps, buf: torch.Tensor):
    """Each member's codes, scales, block offsets and block-list pointers as
    views of the run's buffer (taken after the launch that fills them: the
    host builds them while the kernel runs)."""
    f8, f16, i32 = buf.view(torch.float8_e4m3fn), buf.view(torch.float16), buf.view(torch.int32)
    for p in ps:
        c, s, o, t = p["at"]
        p["codes"] = f8[c:c + p["padded"]]
        p["scales"] = f16[s // 2:s // 2 + p["nblocks"]]
        p["block_off"] = i32[o // 4:o // 4 + p["nblocks"] + 1]
        p["tile_ptr"] = i32[t // 4:t // 4 + p["ntile"]]


def _layout_of(fmt: int, shape, G: int) -> str:
    # e4m3 codes go straight into the layout the fused kernels read; int8
    # codes stay in element order for the reference's compacted stream
    return "tiled" if (fmt == _lib.FMT_E4M3 and tiled_eligible(shape, G)) else "flat"


def _quantize_prepare(fp16_tensor: torch.Tensor, G: int, z_threshold: float, code_format: str, fmt: int) -> dict:
    """Outputs, workspace and aq_quantize arguments of one tensor (numel > 0,
    fp16)."""
    L = _lib.load()
    if G > L.aq_max_block_size():
        raise ValueError(f"block_size {G} exceeds the supported maximum {L.aq_max_block_size()}")
    dev = _lib.compute_device(fp16_tensor.device)
    p = _member_prepare(fp16_tensor, G, fmt, code_format, _layout_of(fmt, fp16_tensor.shape, G), dev)
    ws_bytes = int(L.aq_quantize_workspace_size(p["numel"], G))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    p.update(ws=ws, ws_ptr=ws.data_ptr(), ws_bytes=ws_bytes, stream=_lib.stream_of(dev))
    p["args"] = (p["x"].data_ptr(), p["numel"], G, _threshold_bits(z_threshold), fmt, p["K"],
                 _lib.LAYOUTS[p["layout"]], p["codes"].data_ptr(), p["scales"].data_ptr(), p["block_off"].data_ptr(),
                 ws.data_ptr(), ws_bytes)
    return p


def _finish_outputs(p: dict, nnz: int):
    """The outlier list tensors of a tensor with ``nnz`` outliers (flat
    indices, values, columns) and, for the tiled layout, its block-list
    entries (64 entries of read padding after the last); None otherwise."""
    dev = p["dev"]
    flat_idx = torch.empty(nnz, dtype=torch.int64, device=dev)
    vals = torch.empty(nnz, dtype=torch.float16, device=dev)
    cols = torch.empty(nnz, dtype=torch.int32, device=dev)
    tile_ent = torch.empty(nnz + 64, dtype=torch.int32, device=dev) if p["layout"] == "tiled" else None
    return flat_idx, vals, cols, tile_ent


def _finished_tensor(p: dict, nnz: int, flat_idx, vals, cols, tile_ent, tmax: Optional[DeviceInt]) -> QuantizedTensor:
    """The QuantizedTensor of a tensor whose outlier lists are written (and,
    for int8, its compacted codes, built here); ``tmax`` holds the largest
    block count of the tiled layout's lists (read when first used)."""
    L = _lib.load()
    dev, G, K, N = p["dev"], p["G"], p["K"], p["N"]
    block_off, codes, padded = p["block_off"], p["codes"], p["padded"]
    if K % G == 0:
        # blocks tile the rows, so a row's first outlier is its first block's:
        # the CSR row pointers are every (K / G)-th block offset (per output
        # channel, the block offsets themselves)
        row_ptr = block_off if G == K else block_off[::K // G].contiguous()
    else:
        row_ptr = torch.empty(N + 1, dtype=torch.int32, device=dev)
        _lib.check(L.aq_segment_offsets(_lib.ptr(flat_idx), nnz, N, K, row_ptr.data_ptr(), p["stream"]),
                   "aq_segment_offsets")
    if p["fmt"] == _lib.FMT_INT8:
        fp8_data = torch.empty(padded - nnz, dtype=torch.int8, device=dev)
        _lib.check(L.aq_compact_codes(codes.data_ptr(), padded, _lib.ptr(flat_idx), nnz, _lib.ptr(fp8_data),
                                      p["stream"]), "aq_compact_codes")
    else:
        fp8_data = codes
    p.pop("ws", None)
    extra = {}
    if tile_ent is not None:
        extra = dict(outlier_tile_ptr=p["tile_ptr"], outlier_tile_ent=tile_ent,
                     outlier_tile_max=tmax if nnz else 0)
    qt = QuantizedTensor(
        fp8_data=fp8_data,
        fp16_outliers=vals,
        outlier_indices=flat_idx,
        scale_factors=p["scales"],
        original_shape=p["original_shape"],
        block_size=G,
        code_format=p["code_format"],
        outlier_row_ptr=row_ptr,
        outlier_cols=cols,
        code_layout=p["layout"],
        **extra,
    )
    return qt.to(p["input_device"])


def _quantize_complete(p: dict, nnz: int) -> QuantizedTensor:
    """The outlier lists, CSR rows and block lists of a tensor whose
    aq_quantize has run, given its outlier count: the tiled layout's flat
    list and 16 x 64 block lists in one launch (aq_quantize_finish_tiles),
    the flat list alone otherwise (aq_quantize_finish)."""
    L = _lib.load()
    flat_idx, vals, cols, tile_ent = _finish_outputs(p, nnz)
    args = (p["numel"], p["G"], p["K"], p["block_off"].data_ptr(), nnz, p["ws_ptr"], p["ws_bytes"],
            _lib.ptr(flat_idx), _lib.ptr(vals), _lib.ptr(cols))
    tmax = None
    if tile_ent is not None:
        t = torch.zeros(1, dtype=torch.int32, device=p["dev"])
        _lib.check(L.aq_quantize_finish_tiles(*args, p["tile_ptr"].data_ptr(), tile_ent.data_ptr(), t.data_ptr(),
                                              p["stream"]), "aq_quantize_finish_tiles")
        tmax = DeviceInt(t, 0)
    else:
        _lib.check(L.aq_quantize_finish(*args, p["stream"]), "aq_quantize_finish")
    return _finished_tensor(p, nnz, flat_idx, vals, cols, tile_ent, tmax)


# weights per aq_quantize_grouped launch, most blocks a member may have, and
# most elements a launch may hold (each member's fp16 copy on the device,
# codes and workspace are alive together until its completion)
_QUANT_GROUP_MAX, _QUANT_GROUP_MAX_BLOCKS, _QUANT_GROUP_MAX_ELEMS = 8, 16384, 1 << 28


def _run_launch(tensors, key, z_bits: int, fmt: int, code_format: str) -> dict:
    """Prepare and launch one run of quantize_tensors (members sharing the
    key's device, block size, row length and layout): one workspace for the
    run, one aq_quantize_grouped launch, whose outlier counts (``totals``)
    go to pinned host memory behind it, with an event to wait for them."""
    L = _lib.load()
    arr = _lib.ptr_array
    dev, G, K, layout = key
    # tiled runs (E4M3 codes, the final outputs): every member's
    # count-independent outputs in one allocation, addressed by offset for
    # the launch and viewed after it; flat runs keep their own tensors (int8
    # codes are compacted into new ones)
    buf = None
    if layout == "tiled":
        ps, nbytes = _run_plan(tensors, G, fmt, code_format, dev)
        buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        b0 = buf.data_ptr()
        addr = [tuple(b0 + a for a in p["at"]) for p in ps]
    else:
        ps = [_member_prepare(t, G, fmt, code_format, layout, dev) for t in tensors]
        addr = [(p["codes"].data_ptr(), p["scales"].data_ptr(), p["block_off"].data_ptr(), None) for p in ps]
    n = len(ps)
    ws_bytes = [(int(L.aq_quantize_workspace_size(p["numel"], G)) + 255) // 256 * 256 for p in ps]
    ws = torch.empty(sum(ws_bytes), dtype=torch.uint8, device=dev)
    ws_ptrs, at = [], ws.data_ptr()
    for b in ws_bytes:
        ws_ptrs.append(at)
        at += b
    # [0, n): the outlier counts; [n, 2n): the block lists' largest counts,
    # raised from 0 by the finish
    aux = torch.zeros(2 * n, dtype=torch.int32, device=dev) if layout == "tiled" else \
        torch.empty(n, dtype=torch.int32, device=dev)
    stream = _lib.stream_of(dev)
    numels = arr([p["numel"] for p in ps], ctypes.c_int64)
    offs = arr([a[2] for a in addr])
    ws_ptrs, ws_bytes = arr(ws_ptrs), arr(ws_bytes, ctypes.c_int64)
    _lib.check(L.aq_quantize_grouped(
        n, arr([p["x"].data_ptr() for p in ps]), numels, G, z_bits, fmt, K, _lib.LAYOUTS[layout],
        arr([a[0] for a in addr]), arr([a[1] for a in addr]), offs, ws_ptrs, ws_bytes, aux.data_ptr(), stream),
        "aq_quantize_grouped")
    counts = torch.empty(aux.numel(), dtype=torch.int32, pin_memory=True)
    counts.copy_(aux, non_blocking=True)
    done = torch.cuda.Event()
    done.record(torch.cuda.current_stream(dev))
    if buf is not None:
        _run_views(ps, buf)
    for p, w, b in zip(ps, ws_ptrs, ws_bytes):
        p["ws_ptr"], p["ws_bytes"], p["stream"] = w, b, stream
    return dict(ps=ps, ws=ws, aux=aux, counts=counts, done=done, stream=stream, G=G, K=K, numels=numels, offs=offs,
                ws_ptrs=ws_ptrs, ws_bytes=ws_bytes)


def _run_complete(r: dict) -> list:
    """The QuantizedTensors of a launched run, once its outlier counts are
    on the host: for the tiled layout every member's flat list and block
    lists in one aq_quantize_finish_tiles_grouped launch; one finish per
    member otherwise."""
    ps = r["ps"]
    n = len(ps)
    r["done"].synchronize()
    nnzs = r["counts"].tolist()[:n]
    if ps[0]["layout"] != "tiled":
        return [_quantize_complete(p, nnz) for p, nnz in zip(ps, nnzs)]
    L = _lib.load()
    arr = _lib.ptr_array
    # every member's outlier lists in one allocation: flat indices (int64),
    # values (fp16), columns (int32) and block-list entries (int32, 64 of
    # read padding), addressed by offset for the finish and viewed after it
    at, spans = 0, []
    for nnz in nnzs:
        sp = []
        for nb in (8 * nnz, 2 * nnz, 4 * nnz, 4 * (nnz + 64)):  # indices, values, columns, block-list entries
            sp.append(at)
            at += _a256(nb)
        spans.append(sp)
    lists = torch.empty(at, dtype=torch.uint8, device=r["ps"][0]["dev"])
    b0 = lists.data_ptr()
    nz = lambda a, k: b0 + a if k else None  # noqa: E731  (no address for an empty list)
    aux = r["aux"]
    _lib.check(L.aq_quantize_finish_tiles_grouped(
        n, r["numels"], r["G"], r["K"], r["offs"], arr(nnzs, ctypes.c_int64), r["ws_ptrs"], r["ws_bytes"],
        arr([nz(sp[0], k) for sp, k in zip(spans, nnzs)]), arr([nz(sp[1], k) for sp, k in zip(spans, nnzs)]),
        arr([nz(sp[2], k) for sp, k in zip(spans, nnzs)]), arr([p["tile_ptr"].data_ptr() for p in ps]),
        arr([b0 + sp[3] for sp in spans]), aux.data_ptr() + 4 * n, r["stream"]), "aq_quantize_finish_tiles_grouped")
    r["ws"] = None  # the finish is queued: the workspace may go back to the allocator
    i64, f16, i32 = lists.view(torch.int64), lists.view(torch.float16), lists.view(torch.int32)
    outs = [(i64[sp[0] // 8:sp[0] // 8 + k], f16[sp[1] // 2:sp[1] // 2 + k], i32[sp[2] // 4:sp[2] // 4 + k],
             i32[sp[3] // 4:sp[3] // 4 + k + 64]) for sp, k in zip(spans, nnzs)]
    return [_finished_tensor(p, nnz, *o, DeviceInt(aux, n + k)) for k, (p, nnz, o) in enumerate(zip(ps, nnzs, outs))]


def quantize_tensors(tensors, block_size: int = 128, z_threshold: float = 3.0, *,
                     code_format: str = DEFAULT_CODE_FORMAT):
    """``[quantize_tensor(t, ...) for t in tensors]``, bit for bit, with
    the tensors that share a device, a block size, a row length and a code
    layout (and have at most 16384 blocks) quantized by one launch per run
    of up to 8 (aq_quantize_grouped, at most 2^28 elements a run): the small
    weights of a layer then share the GPU instead of each filling one round
    of it, and each run costs one host sync, taken once the next run is
    queued (two runs are in flight at a time).  Tensors with more blocks are
    quantized one at a time, each completed before the next is prepared.
    The members of a tiled run share two allocations (their codes, scales,
    offsets and block-list pointers; their outlier lists), so a run's device
    memory goes back to the allocator when the last of its QuantizedTensors
    does."""
    fmt = _format_id(code_format)
    out = [None] * len(tensors)
    groups = {}
    L = None
    for i, t in enumerate(tensors):
        if not isinstance(t, torch.Tensor) or t.dtype != torch.float16 or t.numel() == 0:
            out[i] = quantize_tensor(t, block_size, z_threshold, code_format=code_format)
            continue
        G = _resolve_block(block_size, t.shape)
        if (t.numel() + G - 1) // G > _QUANT_GROUP_MAX_BLOCKS:
            out[i] = quantize_tensor(t, block_size, z_threshold, code_format=code_format)
            continue
        if L is None:
            L = _lib.load()
        if G > L.aq_max_block_size():
            raise ValueError(f"block_size {G} exceeds the supported maximum {L.aq_max_block_size()}")
        key = (_lib.compute_device(t.device), G, _rows_cols(t.shape)[1], _layout_of(fmt, t.shape, G))
        groups.setdefault(key, []).append(i)
    runs = []
    for key, idx in groups.items():
        run, elems = [], 0
        for i in idx:
            n = tensors[i].numel()
            if run and (len(run) == _QUANT_GROUP_MAX or elems + n > _QUANT_GROUP_MAX_ELEMS):
                runs.append((key, run))
                run, elems = [], 0
            run.append(i)
            elems += n
        if run:
            runs.append((key, run))
    z_bits = _threshold_bits(z_threshold)
    inflight = None  # the run launched last, completed once the next one is queued
    for key, run in runs:
        r = _run_launch([tensors[i] for i in run], key, z_bits, fmt, code_format)
        r["run"] = run
        # the host waits for a run's outlier counts only after queueing the
        # next run, so that run's kernel runs while this one is finished
        if inflight is not None:
            for i, qt in zip(inflight["run"], _run_complete(inflight)):
                out[i] = qt
        inflight = r
    if inflight is not None:
        for i, qt in zip(inflight["run"], _run_complete(inflight)):
            out[i] = qt
    return out


def _stored_codes(q: QuantizedTensor, device: torch.device) -> torch.Tensor:
    """The dense codes as stored (flat or tiled), expanding the int8
    compacted stream."""
    numel = q.original_shape.numel()
    G = q.block_size
    padded = (numel + G - 1) // G * G
    if q.code_format != "int8":
        return q.fp8_data.view(torch.uint8)
    L = _lib.load()
    dense = torch.empty(padded, dtype=torch.uint8, device=device)
    nnz = q.outlier_indices.numel()
    _lib.check(L.aq_expand_codes(_lib.ptr(q.fp8_data), padded, _lib.ptr(q.outlier_indices), nnz,
                                 dense.data_ptr(), _lib.stream_of(device)), "aq_expand_codes")
    return dense


def dense_codes(qt: QuantizedTensor, device: torch.device) -> torch.Tensor:
    """One uint8 code per element of the padded tensor in element order, 0 at
    outliers, on ``device`` (expands the int8 stream, untiles tiled codes)."""
    q = qt.to(device)
    codes = _stored_codes(q, device)
    if q.code_layout != "tiled":
        return codes
    L = _lib.load()
    N, K = _rows_cols(q.original_shape)
    flat = torch.empty_like(codes)
    _lib.check(L.aq_untile_codes(codes.data_ptr(), N, K, flat.data_ptr(), _lib.stream_of(device)), "aq_untile_codes")
    return flat


def kernel_codes(qt: QuantizedTensor, device: torch.device) -> torch.Tensor:
    """Codes in the tiled layout the quantized-linear kernels read (a view of
    fp8_data when it is stored tiled, else a tiled copy)."""
    q = qt.to(device)
    if not tiled_eligible(q.original_shape, q.block_size):
        raise ValueError(f"shape {tuple(q.original_shape)} with block {q.block_size} does not tile")
    codes = _stored_codes(q, device)
    if q.code_layout == "tiled":
        return codes
    L = _lib.load()
    N, K = _rows_cols(q.original_shape)
    tiled = torch.empty_like(codes)
    _lib.check(L.aq_tile_codes(codes.data_ptr(), N, K, tiled.data_ptr(), _lib.stream_of(device)), "aq_tile_codes")
    return tiled


def tiles_eligible(shape) -> bool:
    """Whether the outliers of a weight of this shape can be listed per
    16 x 64 block (2-D view [N, K] with N % 16 == 0, K % 64 == 0)."""
    if len(shape) < 2:
        return False
    N, K = _rows_cols(shape)
    return N >= 16 and N % 16 == 0 and K >= 64 and K % 64 == 0


def build_outlier_tiles(qt: QuantizedTensor, device: torch.device, lazy_max: bool = False):
    """(tile_ptr, tile_ent, tile_max): the outliers of ``qt`` per block of 16
    rows x 64 columns (aq_outlier_tiles), from its CSR lists, on ``device``,
    and the largest count in one block (one host sync, or with ``lazy_max`` a
    DeviceInt read when first used)."""
    q = qt.to(device)
    if not tiles_eligible(q.original_shape) or q.outlier_row_ptr is None:
        raise ValueError(f"shape {tuple(q.original_shape)} has no 16 x 64 outlier blocks")
    L = _lib.load()
    N, K = _rows_cols(q.original_shape)
    nnz = q.fp16_outliers.numel()
    tile_ptr = torch.empty((N // 16) * (K // 64) + 1, dtype=torch.int32, device=device)
    tile_ent = torch.empty(nnz + 64, dtype=torch.int32, device=device)  # + 64 entries of read padding (zeroed)
    tmax = torch.zeros(1, dtype=torch.int32, device=device)  # raised to the largest block's count
    _lib.check(L.aq_outlier_tiles(q.outlier_row_ptr.data_ptr(), _lib.ptr(q.outlier_cols), _lib.ptr(q.fp16_outliers),
                                  N, K, tile_ptr.data_ptr(), tile_ent.data_ptr(), tmax.data_ptr(),
                                  _lib.stream_of(device)),
               "aq_outlier_tiles")
    if not nnz:
        return tile_ptr, tile_ent, 0
    return tile_ptr, tile_ent, DeviceInt(tmax[0]) if lazy_max else int(tmax.item())


def outlier_tiles(qt: QuantizedTensor, device: torch.device):
    """(tile_ptr, tile_ent, tile_max) of ``qt`` on ``device``: the stored
    block outlier lists, or built from the CSR lists."""
    if qt.outlier_tile_ptr is not None:
        return qt.outlier_tile_ptr.to(device), qt.outlier_tile_ent.to(device), qt.outlier_tile_max
    return build_outlier_tiles(qt, device)


# --- Dequantization cache (reference :153-154): id(QuantizedTensor) -> fp16 tensor.
# Each entry also holds the QuantizedTensor it was computed from: while the
# entry exists that object stays alive, so its id cannot be handed to another
# object, and a lookup by id can never return another tensor's weights (the
# reference, which stores only the fp16 tensor, can: ids are reused after
# garbage collection).  The reference's API is unchanged: keys are ids, and
# clear_dequantized_cache(id) / clear_dequantized_cache() drop entries.
_dequantized_weights_cache = {}
_cache_lock = threading.Lock()


def dequantize_tensor(quant_data: QuantizedTensor, target_device: torch.device) -> torch.Tensor:
    """Rebuild the fp16 tensor on ``target_device`` (reference :156-251):
    fp16(code * scale) for non-outliers, outlier values verbatim.  Memoised by
    the identity of ``quant_data`` like the reference."""
    target_device = torch.device(target_device)
    if target_device.type == "cuda" and target_device.index is None:
        target_device = torch.device("cuda", torch.cuda.current_device())
    cache_key = id(quant_data)
    with _cache_lock:
        entry = _dequantized_weights_cache.get(cache_key)
        if entry is not None and entry[0] is quant_data:
            cached = entry[1]
            if cached.device != target_device:
                cached = cached.to(target_device)
                _dequantized_weights_cache[cache_key] = (quant_data, cached)
            return cached

    numel = quant_data.original_shape.numel()
    if numel == 0:
        final = torch.zeros(quant_data.original_shape, dtype=torch.float16, device=target_device)
    else:
        L = _lib.load()
        dev = _lib.compute_device(target_device)
        q = quant_data.to(dev)
        fmt = _format_id(q.code_format)
        codes = _stored_codes(q, dev)
        _, K = _rows_cols(q.original_shape)
        out = torch.empty(numel, dtype=torch.float16, device=dev)
        nnz = q.outlier_indices.numel()
        _lib.check(L.aq_dequantize(codes.data_ptr(), q.scale_factors.data_ptr(), numel, q.block_size, fmt, K,
                                   _lib.LAYOUTS[q.code_layout], _lib.ptr(q.outlier_indices),
                                   _lib.ptr(q.fp16_outliers), nnz, out.data_ptr(), _lib.stream_of(dev)),
                   "aq_dequantize")
        final = out.view(q.original_shape).to(target_device)

    with _cache_lock:
        _dequantized_weights_cache[cache_key] = (quant_data, final)
    return final


def discard_dequantized(quant_data_id: int) -> None:
    """Drop the cached fp16 copy of one QuantizedTensor (by id), without
    returning the allocator's cached blocks to the device (the per-layer
    counterpart of clear_dequantized_cache for code that runs every step)."""
    with _cache_lock:
        _dequantized_weights_cache.pop(quant_data_id, None)


def clear_dequantized_cache(quant_data_id=None):
    """Clear one entry (by id) or the whole cache (reference :253-263)."""
    global _dequantized_weights_cache
    with _cache_lock:
        if quant_data_id is not None and quant_data_id in _dequantized_weights_cache:
            del _dequantized_weights_cache[quant_data_id]
        elif quant_data_id is None:
            _dequantized_weights_cache = {}
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
