"""QuantizedLinear: an nn.Linear replacement whose weight stays quantized.

Same interface as the reference class
(/root/reference/integration/atlas_wrappers.py:21-83; also importable as
``integration.atlas_wrappers.QuantizedLinear``): constructor
``(quantized_weights, bias)``, plain attributes ``quantized_weights``,
``bias`` and ``original_shape``, ``forward(x)`` with F.linear semantics over
any leading dimensions, the same ``extra_repr``.

The reference's forward dequantizes the whole weight to fp16 (cached) and
calls F.linear (:56,67).  Here forward is one launch of the fused
dequant-GEMV / dequant-GEMM (``aq_qlinear``): the codes are decoded in
registers and never written back as fp16.  Weights that do not tile
(out_features % 16, in_features % 128, or a block size that is not a
multiple of 32 dividing in_features) take the dequantize kernel followed by
F.linear on the GPU.

``AtlasAttentionWrapper`` (reference :84-262) keeps an attention module's
key/value history in a UnifiedMemoryManager (tiered KV cache).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _lib
from ..quant.adaptive_quantizer import (QuantizedTensor, _format_id, _rows_cols, dequantize_tensor, kernel_codes,
                                        outlier_tiles, tiled_eligible)


GEMV_MAX_M = 64  # aq_qlinear runs the dequant-GEMV up to this many rows of x
# from this many rows of x on, calls pass the outlier block lists: the
# shared-x GEMV (6 <= M <= 64) adds the outliers with MFMAs from them
LISTS_MIN_M = 6
# from this many rows on, calls pass the workspace too: given the lists the
# library runs the GEMM for grids too short for the GEMV (and always past
# GEMV_MAX_M)
GEMM_MIN_M = 33


def _workspace(M: int, Ns, K: int, dev: torch.device):
    """The GEMM's split-K workspace (None when the call needs none) and its size."""
    if M < GEMM_MIN_M:
        return None, 0
    # one query for the whole group: the library plans a grouped call over
    # all its output columns, and returns 0 when it runs the GEMV
    n = int(_lib.load().aq_qlinear_workspace_size(M, sum(Ns), K))
    if n == 0:
        return None, 0
    return torch.empty(n, dtype=torch.uint8, device=dev), n


def fused_supported(qt: QuantizedTensor) -> bool:
    """The fused kernels need 16-row x 128-column tiles and blocks of a
    multiple of 32 that divide the row."""
    return qt.outlier_row_ptr is not None and tiled_eligible(qt.original_shape, qt.block_size)


def qlinear_grouped(x: torch.Tensor, qts, biases=None, codes=None, tiles=None):
    """[x W_i^T + b_i for each quantized W_i] in one launch; all W_i share
    in_features (aq_qlinear_grouped).  ``codes`` may carry the tiled code
    arrays and ``tiles`` the (tile_ptr, tile_ent, tile_max) outlier block
    lists (saves rebuilding them per call for weights that do not store
    them)."""
    dev = x.device
    L = _lib.load()
    n = len(qts)
    if not 1 <= n <= _lib.MAX_GROUP:
        raise ValueError(f"1..{_lib.MAX_GROUP} weights per grouped call, got {n}")
    K = int(qts[0].original_shape[-1])
    fmt = qts[0].code_format
    for q in qts:
        if int(q.original_shape[-1]) != K or q.code_format != fmt or not fused_supported(q):
            raise ValueError("grouped weights must share in_features and code format and tile")
    biases = list(biases) if biases is not None else [None] * n
    codes = list(codes) if codes is not None else [kernel_codes(q, dev) for q in qts]
    x2 = x.reshape(-1, K)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    M = x2.shape[0]
    Ns = [_rows_cols(q.original_shape)[0] for q in qts]
    ys = [torch.empty((M, N), dtype=torch.float16, device=dev) for N in Ns]
    if M > 0:
        arr = _lib.ptr_array
        if M >= LISTS_MIN_M:
            tiles = list(tiles) if tiles is not None else [outlier_tiles(q, dev) for q in qts]
        else:
            tiles = [(None, None, 0)] * n
        ws, ws_bytes = _workspace(M, Ns, K, dev)
        _lib.check(L.aq_qlinear_grouped(
            x2.data_ptr(), M, K, _format_id(fmt), n, arr(Ns, ctypes.c_int64), arr([c.data_ptr() for c in codes]),
            arr([q.scale_factors.data_ptr() for q in qts]), arr([q.block_size for q in qts], ctypes.c_int64),
            arr([q.outlier_row_ptr.data_ptr() for q in qts]), arr([_lib.ptr(q.outlier_cols) for q in qts]),
            arr([_lib.ptr(q.fp16_outliers) for q in qts]), arr([_lib.ptr(t[0]) for t in tiles]),
            arr([_lib.ptr(t[1]) for t in tiles]), arr([t[2] for t in tiles], ctypes.c_int64),
            arr([_lib.ptr(b) for b in biases]),
            arr([y.data_ptr() for y in ys]), _lib.ptr(ws), ws_bytes, _lib.stream_of(dev)), "aq_qlinear_grouped")
    return [y.view(*x.shape[:-1], N) for y, N in zip(ys, Ns)]


PRO_NONE, PRO_RMS, PRO_LAYERNORM, PRO_SWIGLU = 0, 1, 2, 3


def qlinear_decode(x: torch.Tensor, qts, biases, codes, prologue: int = PRO_NONE, x2=None, norm_weight=None,
                   norm_bias=None, eps: float = 0.0, residuals=None, relu=None, tiles=None, swiglu_pair=False):
    """One launch of aq_qlinear_decode: [f(x) W_i^T + b_i] for up to 4
    quantized W_i sharing in_features, x of M rows (1, or 6..64), where f is
    the prologue (none, RMSNorm / LayerNorm with ``norm_weight`` /
    ``norm_bias`` and ``eps`` -- M = 1 only --, or the SwiGLU product
    silu(x) * x2; every prologue needs M = 1), each output optionally passed
    through ReLU (``relu[i]``) and added to ``residuals[i]`` (fp16 [M,
    N_i]).  ``codes`` are the weights' tiled code arrays, ``tiles`` their
    (tile_ptr, tile_ent, tile_max) outlier block lists (built when not
    given, used from LISTS_MIN_M rows on).  ``swiglu_pair``: qts are (gate,
    up) and the result is [fp16(fp16(silu(x W_g^T)) (x W_u^T))], one
    output (6 <= M <= 64)."""
    dev = x.device
    L = _lib.load()
    n = len(qts)
    K = int(qts[0].original_shape[-1])
    fmt = qts[0].code_format
    for q in qts:
        if int(q.original_shape[-1]) != K or q.code_format != fmt or not fused_supported(q):
            raise ValueError("qlinear_decode: weights must share in_features and code format and tile")
    xs = [x.reshape(-1, K)] + ([x2.reshape(-1, K)] if x2 is not None else [])
    M = xs[0].shape[0]
    for t in xs:
        if t.shape[0] != M or not t.is_contiguous() or t.data_ptr() % 16 or t.dtype != torch.float16:
            raise ValueError("qlinear_decode: x (and x2) must be contiguous, 16-byte aligned fp16 [M, K]")
    Ns = [_rows_cols(q.original_shape)[0] for q in qts]
    ys = [torch.empty((M, N), dtype=torch.float16, device=dev) for N in (Ns[:1] if swiglu_pair else Ns)]
    arr = _lib.ptr_array
    res = None if residuals is None else arr([_lib.ptr(r) for r in residuals])
    yp = [y.data_ptr() for y in ys]
    if swiglu_pair:
        if n != 2 or Ns[0] != Ns[1]:
            raise ValueError("qlinear_decode: a SwiGLU pair is two weights (gate, up) of equal out_features")
        acts = arr([2, 0], ctypes.c_int32)
        yp = [yp[0], yp[0]]  # the one output; up's is never written
    else:
        acts = None if relu is None else arr([int(bool(r)) for r in relu], ctypes.c_int32)
    if M >= LISTS_MIN_M:
        tiles = list(tiles) if tiles is not None else [outlier_tiles(q, dev) for q in qts]
        tps, tes = arr([t[0].data_ptr() for t in tiles]), arr([t[1].data_ptr() for t in tiles])
    else:
        tps = tes = None
    _lib.check(L.aq_qlinear_decode(
        xs[0].data_ptr(), M, K, _format_id(fmt), n, arr(Ns, ctypes.c_int64), arr([c.data_ptr() for c in codes]),
        arr([q.scale_factors.data_ptr() for q in qts]), arr([q.block_size for q in qts], ctypes.c_int64),
        arr([q.outlier_row_ptr.data_ptr() for q in qts]), arr([_lib.ptr(q.outlier_cols) for q in qts]),
        arr([_lib.ptr(q.fp16_outliers) for q in qts]), tps, tes, arr([_lib.ptr(b) for b in biases]),
        arr(yp), int(prologue), None if x2 is None else xs[1].data_ptr(), _lib.ptr(norm_weight),
        _lib.ptr(norm_bias), ctypes.c_float(eps), res, acts, _lib.stream_of(dev)), "aq_qlinear_decode")
    return ys


def qlinear(x: torch.Tensor, qt: QuantizedTensor, bias: Optional[torch.Tensor],
            codes: Optional[torch.Tensor] = None, tiles=None) -> torch.Tensor:
    """y = x W^T + b for W in quantized form, through aq_qlinear.  ``codes``
    may carry the tiled code array and ``tiles`` the outlier block lists."""
    dev = x.device
    K = int(qt.original_shape[-1])
    N = qt.original_shape.numel() // K
    x2 = x.reshape(-1, K)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    M = x2.shape[0]
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    if M == 0:
        return y.view(*x.shape[:-1], N)
    if codes is None:
        codes = kernel_codes(qt, dev)
    tp, te, tmax = (tiles if tiles is not None else outlier_tiles(qt, dev)) if M >= LISTS_MIN_M else (None, None, 0)
    L = _lib.load()
    ws, ws_bytes = _workspace(M, [N], K, dev)
    _lib.check(L.aq_qlinear(x2.data_ptr(), M, K, N, codes.data_ptr(), qt.scale_factors.data_ptr(), qt.block_size,
                            _format_id(qt.code_format), qt.outlier_row_ptr.data_ptr(), _lib.ptr(qt.outlier_cols),
                            _lib.ptr(qt.fp16_outliers), _lib.ptr(tp), _lib.ptr(te), tmax, _lib.ptr(bias), y.data_ptr(),
                            _lib.ptr(ws), ws_bytes, _lib.stream_of(dev)), "aq_qlinear")
    return y.view(*x.shape[:-1], N)


class SiblingGroup:
    """QuantizedLinear modules that a model calls one after another on the
    same input (q/k/v projections, gate/up): at decode sizes the first
    member's forward runs one grouped launch for all of them and keeps the
    other outputs for their own forward on that very tensor object (same
    object, unchanged version); any other input computes as usual.  A kept
    output lives until its member consumes it or the group runs again."""

    def __init__(self, members):
        self.members = list(members)
        self.x = None
        self.version = -1
        self.out = {}

    def _prepare(self, dev, lists: bool):
        """The grouped call's fixed arguments for the members' current
        weights and biases on ``dev`` (rebuilt when any of them changes);
        ``lists``: with the outlier block lists (calls of LISTS_MIN_M rows or
        more), else without them (none are built)."""
        qs, biases, codes = [], [], []
        for m in self.members:
            q = m._weights_on(dev)
            m._ensure_codes(q, dev)
            qs.append(q)
            biases.append(m.bias)
            codes.append(m._codes)
        key = (dev, tuple(id(q) for q in qs), tuple(id(b) for b in biases), lists)
        p = getattr(self, "_prep", None)
        if p is not None and p[0] == key:
            return p
        arr, n = _lib.ptr_array, len(qs)
        K = int(qs[0].original_shape[-1])
        Ns = [_rows_cols(q.original_shape)[0] for q in qs]
        tiles = ([m._ensure_tiles(q, dev) for m, q in zip(self.members, qs)] if lists
                 else [(None, None, 0)] * n)
        # no tile_max: calls below GEMM_MIN_M rows always take a GEMV
        fixed = (_format_id(qs[0].code_format), n, arr(Ns, ctypes.c_int64), arr([c.data_ptr() for c in codes]),
                 arr([q.scale_factors.data_ptr() for q in qs]), arr([q.block_size for q in qs], ctypes.c_int64),
                 arr([q.outlier_row_ptr.data_ptr() for q in qs]), arr([_lib.ptr(q.outlier_cols) for q in qs]),
                 arr([_lib.ptr(q.fp16_outliers) for q in qs]), arr([_lib.ptr(t[0]) for t in tiles]),
                 arr([_lib.ptr(t[1]) for t in tiles]), None, arr([_lib.ptr(b) for b in biases]))
        # the tuple keeps the weights, biases, codes and block lists its addresses point into
        self._prep = p = (key, K, Ns, fixed, (qs, biases, codes, tiles))
        return p

    def run(self, leader, x):
        dev = x.device
        K = int(x.shape[-1])
        _, K, Ns, fixed, _keep = self._prepare(dev, x.numel() // K >= LISTS_MIN_M)
        x2 = x.reshape(-1, K)
        if not x2.is_contiguous() or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        M = x2.shape[0]
        buf = torch.empty(M * sum(Ns), dtype=torch.float16, device=dev)
        ys, off = [], 0
        for N in Ns:  # each output a contiguous [M, N] piece of one allocation
            ys.append(buf[off:off + M * N].view(M, N))
            off += M * N
        _lib.check(_lib.load().aq_qlinear_grouped(x2.data_ptr(), M, K, *fixed,
                                                  _lib.ptr_array([y.data_ptr() for y in ys]), None, 0,
                                                  _lib.stream_of(dev)), "aq_qlinear_grouped")
        ys = [y.view(*x.shape[:-1], N) for y, N in zip(ys, Ns)]
        self.x, self.version = x, x._version
        self.out = {id(m): y for m, y in zip(self.members, ys) if m is not leader}
        return ys[self.members.index(leader)]

    def take(self, member, x):
        if self.x is x and x._version == self.version:
            y = self.out.pop(id(member), None)
            if not self.out:
                self.x = None
            return y
        return None


class QuantizedLinear(nn.Module):
    """A Linear layer that uses a QuantizedTensor for weights."""

    def __init__(self, quantized_weights: QuantizedTensor, bias: Optional[torch.Tensor]):
        super().__init__()
        self.quantized_weights = quantized_weights
        self.bias = bias
        self.original_shape = getattr(quantized_weights, "original_shape", None)
        # derived from the weight object _derived_from on its device: the tiled
        # codes (int8: expanded and tiled once) and the outlier block lists
        self._derived_from = None
        self._codes = None
        self._tiles = None
        # the GEMV call's fixed arguments, valid while device, weight and bias
        # objects stay the same: (device, bias, weight, K, N, entry, args, codes)
        self._prep = None
        self._group = None  # SiblingGroup this module leads or follows (decode-time grouped launch)

    def _weights_on(self, device: torch.device) -> QuantizedTensor:
        q = self.quantized_weights
        if not hasattr(q, "fp8_data"):
            raise TypeError(f"Weight in QuantizedLinear ({id(self)}) is not a valid QuantizedTensor: {type(q)}")
        if q.fp8_data.device != device:
            self.quantized_weights = q = q.to(device)
            self._codes = None
            self._tiles = None
            self._prep = None
        if self.bias is not None and self.bias.device != device:
            self.bias = self.bias.to(device)
        return q

    def _set_weights(self, q: QuantizedTensor, bias: Optional[torch.Tensor]) -> None:
        """Assign weight and bias, dropping everything derived from the
        previous ones (codes, block lists, prepared arguments, the sibling
        group's prepared call and kept outputs)."""
        self.quantized_weights = q
        self.bias = bias
        self._derived_from = self._codes = self._tiles = self._prep = None
        g = self._group
        if g is not None:
            g._prep = None
            g.out = {}
            g.x = None

    def _ensure_codes(self, q: QuantizedTensor, dev: torch.device) -> None:
        if self._derived_from is not q:  # a weight assigned since (q is on dev here)
            self._derived_from, self._codes, self._tiles = q, None, None
        if self._codes is None or self._codes.device != dev:
            self._codes = kernel_codes(q, dev)

    def _ensure_tiles(self, q: QuantizedTensor, dev: torch.device):
        """The weight's outlier block lists on ``dev`` (stored ones, or built
        once and kept); after _ensure_codes(q, dev)."""
        if self._tiles is None or self._tiles[0].device != dev:
            self._tiles = outlier_tiles(q, dev)
        return self._tiles

    def _grouped_forward(self, x: torch.Tensor) -> Optional[torch.Tensor]:
        g = self._group
        y = g.take(self, x)
        if y is not None:
            return y
        # an inference tensor has no version counter, so a kept output could
        # not be matched to an unmodified input: such inputs compute alone
        if (g.members[0] is self and not x.is_inference() and x.dtype == torch.float16 and x.device.type == "cuda"
                and 0 < x.numel() < GEMM_MIN_M * x.shape[-1]
                and all(fused_supported(m.quantized_weights) for m in g.members)):
            return g.run(self, x)
        return None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if torch.is_grad_enabled() and (x.requires_grad or (self.bias is not None and self.bias.requires_grad)):
            # the fused kernels record no autograd graph: inputs that need
            # gradients take the reference's own computation, F.linear on the
            # dequantized weight (atlas_wrappers.py:56,67), whose backward
            # reaches x and the bias
            return self._forward_reference(x)
        if self._group is not None:
            y = self._grouped_forward(x)
            if y is not None:
                return y
        # decode fast path (M < GEMM_MIN_M rows of x): one library call with
        # the weight's arguments prepared by an earlier forward on this device
        p = self._prep
        if (p is not None and x.dtype == torch.float16 and self.bias is p[1] and self.quantized_weights is p[2]
                and x.device == p[0] and x.shape[-1] == p[3]):
            K, N = p[3], p[4]
            x2 = x.reshape(-1, K)
            M = x2.shape[0]
            # from LISTS_MIN_M rows on the GEMV wants the outlier block lists:
            # arguments prepared without them (an earlier call with fewer
            # rows) go through _forward, which builds them once
            if 0 < M < GEMM_MIN_M and (M < LISTS_MIN_M or p[8] is not None):
                if not x2.is_contiguous() or x2.data_ptr() % 16:
                    x2 = x2.contiguous()
                y = torch.empty((M, N), dtype=torch.float16, device=p[0])
                _lib.check(p[5](x2.data_ptr(), M, K, N, *p[6], y.data_ptr(), None, 0, _lib.stream_of(p[0])),
                           "aq_qlinear")
                return y.view(*x.shape[:-1], N)
        return self._forward(x)

    def _checked_weights(self, x: torch.Tensor) -> QuantizedTensor:
        dev = x.device
        if dev.type != "cuda":
            raise RuntimeError(f"QuantizedLinear runs on a HIP device; input is on {dev}")
        q = self._weights_on(dev)
        if x.dtype != torch.float16:
            raise RuntimeError(f"expected both mat1 and mat2 to have the same dtype, but got: {x.dtype} != Half")
        K = int(q.original_shape[-1])
        if x.shape[-1] != K:
            raise RuntimeError(f"mat1 and mat2 shapes cannot be multiplied (input last dim {x.shape[-1]} vs "
                               f"in_features {K})")
        return q

    def _forward_reference(self, x: torch.Tensor) -> torch.Tensor:
        q = self._checked_weights(x)
        return F.linear(x, dequantize_tensor(q, x.device), self.bias)

    def _forward(self, x: torch.Tensor) -> torch.Tensor:
        dev = x.device
        q = self._checked_weights(x)
        K = int(q.original_shape[-1])
        if not fused_supported(q):
            return F.linear(x, dequantize_tensor(q, dev), self.bias)
        self._ensure_codes(q, dev)
        M = x.numel() // K if K else 0
        if M >= LISTS_MIN_M:
            self._ensure_tiles(q, dev)
        elif self._tiles is not None and self._tiles[0].device != dev:
            self._tiles = None
        # block lists only once a call has enough rows to use them: fewer rows
        # (decode at batch 1) never build them, which would cost a host sync
        # per call for weights streamed in without stored lists
        tiles = self._tiles
        p = self._prep
        if p is None or p[0] != dev or p[1] is not self.bias or p[2] is not q or (tiles is not None and p[8] is None):
            N = q.original_shape.numel() // K
            tp, te = (None, None) if tiles is None else tiles[:2]
            # the tuple holds the codes, block lists, weight and bias objects
            # its addresses point into (no tile_max: the fast path's calls
            # always take a GEMV)
            self._prep = (dev, self.bias, q, K, N, _lib.load().aq_qlinear,
                          (self._codes.data_ptr(), q.scale_factors.data_ptr(), q.block_size,
                           _format_id(q.code_format), q.outlier_row_ptr.data_ptr(), _lib.ptr(q.outlier_cols),
                           _lib.ptr(q.fp16_outliers), _lib.ptr(tp), _lib.ptr(te), 0, _lib.ptr(self.bias)),
                          self._codes, tiles)
        return qlinear(x, q, self.bias, self._codes, tiles)

    def _apply(self, fn, recurse=True):
        # module.to(device) / .cuda() also moves the quantized weight and the
        # bias (plain attributes, invisible to nn.Module); dtype casts leave
        # the codes alone.
        super()._apply(fn, recurse)
        probe = fn(torch.empty(0, dtype=torch.float16, device=self._current_device()))
        if probe.device != self._current_device():
            self._weights_on(probe.device)
        return self

    def _current_device(self) -> torch.device:
        q = self.quantized_weights
        return q.fp8_data.device if hasattr(q, "fp8_data") else torch.device("cpu")

    def extra_repr(self) -> str:
        q_shape, q_device = None, "N/A"
        if hasattr(self, "quantized_weights") and self.quantized_weights:
            q_shape = self.original_shape
            try:
                q_device = self.quantized_weights.fp8_data.device
            except AttributeError:
                pass
        return f"quantized_shape={q_shape}, bias={self.bias is not None}, device={q_device}"


class AtlasAttentionWrapper(nn.Module):
    """An attention module whose key/value history lives in a
    UnifiedMemoryManager (reference :84-262).

    Constructor as the reference's: ``(q_proj, k_proj, v_proj, o_proj,
    parent_layer, memory_manager, layer_idx, model_type)``.  The wrapped
    module is the decoder layer's own attention (``parent_layer.self_attn``),
    whose forward still does the projections (QuantizedLinear after the
    swap), the rotary embedding, the masks and the attention itself; the
    wrapper makes the HF cache it is handed keep this layer's keys and
    values in the manager (``KVCacheLayer``: appended in place in HBM,
    demoted to host memory or disk when the manager's limits say so).  A new
    cache object starts the layer's history afresh.

    Unlike the reference's, which recomputed attention itself: the rotary
    embedding is applied to the new positions only (the reference applied
    it again to the whole concatenated history each step), the causal mask
    of a prompt is kept, OPT's query scaling is applied once, and Llama's
    ``o_proj`` is found as well as OPT's ``out_proj``.  Results equal the
    unwrapped model's on the same inputs."""

    def __init__(self, q_proj: nn.Module, k_proj: nn.Module, v_proj: nn.Module, o_proj: nn.Module,
                 parent_layer: nn.Module, memory_manager, layer_idx: int, model_type: str):
        super().__init__()
        inner = getattr(parent_layer, "self_attn", None)
        if inner is None or not all(p is not None for p in (q_proj, k_proj, v_proj, o_proj)):
            raise ValueError(f"CRITICAL: no attention module or projections in layer {layer_idx}")
        # the wrapped module's children under their own names (state-dict keys
        # unchanged); the module itself stays outside the module tree
        for name, child in inner.named_children():
            setattr(self, name, child)
        object.__setattr__(self, "_inner", inner)
        self.memory_manager = memory_manager
        self.layer_idx = layer_idx
        self.model_type = model_type
        self._bound = None  # the HF cache whose layer entry is the manager's

    def _bind(self, cache) -> None:
        from ..memory.unified_memory_manager import KVCacheLayer
        idx = getattr(self._inner, "layer_idx", self.layer_idx)
        layers = getattr(cache, "layers", None)
        if layers is None:
            raise TypeError(f"AtlasAttentionWrapper: unsupported cache type {type(cache).__name__}")
        while len(layers) <= idx:
            layers.append(cache.layer_class_to_replicate())
        cur = layers[idx]
        if isinstance(cur, KVCacheLayer) and cur.manager is self.memory_manager:
            return
        if getattr(cur, "is_sliding", False):
            raise NotImplementedError("AtlasAttentionWrapper: sliding-window cache layers are not supported")
        self.memory_manager.reset_layer(idx)  # a new cache: a new history
        layers[idx] = KVCacheLayer(self.memory_manager, idx)

    def forward(self, hidden_states, *args, **kwargs):
        for key in ("past_key_values", "past_key_value"):
            cache = kwargs.get(key)
            if cache is not None:
                if cache is not self._bound:
                    self._bind(cache)
                    self._bound = cache
                break
        return self._inner(hidden_states, *args, **kwargs)
