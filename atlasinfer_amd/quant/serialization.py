"""Quantized weights on disk: safetensors files of QuantizedTensor fields.

The reference has no stored form for its quantized weights: every run loads
the fp16 checkpoint and quantizes each Linear again
(/root/reference/examples/run_atlas_inference.py:173-180, through
integration/model_modifier.py:95-143), and ``QuantizedTensor``
(atlasinfer_core/quant/adaptive_quantizer.py:8-42) lives only in memory.
This module stores what ``quantize_tensor`` produced so a later run skips the
quantize pass:

* ``save_quantized(tensors, path)`` / ``load_quantized(path, device)`` -- a
  dict of named QuantizedTensors (plus optional named plain tensors such as
  biases).
* ``save_quantized_model(model, path)`` / ``load_quantized_model(model, path)``
  -- every ``QuantizedLinear`` of a model with its bias; loading swaps the
  modules of a freshly built model (e.g. ``from_config``) for QuantizedLinear
  ones holding the stored weights, as ``apply_atlas_quantization_to_model``
  would have after quantizing.

File layout: one safetensors file.  Tensor ``"<name>/<field>"`` for every
tensor field of a QuantizedTensor that is not None (codes keep their dtype:
int8 for the reference's compacted stream, float8_e4m3fn for E4M3), and
``"<name>"`` for a plain tensor.  The header metadata holds ``format``
(``"atlasinfer_amd.quantized"``), ``version`` and ``entries``: JSON mapping
each quantized name to its non-tensor fields (original_shape, block_size,
code_format, code_layout, outlier_tile_max).  Loading uses safetensors only
(no pickle); a file whose header or tensors disagree with the format raises
ValueError before any module is touched.
"""
from __future__ import annotations

import json
from typing import Dict, Mapping, Optional, Tuple

import torch
import torch.nn as nn
from safetensors import safe_open
from safetensors.torch import save_file

from .adaptive_quantizer import QuantizedTensor, tiled_eligible, tiles_eligible

FORMAT_NAME = "atlasinfer_amd.quantized"
FORMAT_VERSION = 1

_TENSOR_FIELDS = ("fp8_data", "fp16_outliers", "outlier_indices", "scale_factors", "outlier_row_ptr",
                  "outlier_cols", "outlier_tile_ptr", "outlier_tile_ent")
_REQUIRED = ("fp8_data", "fp16_outliers", "outlier_indices", "scale_factors")
_CODE_DTYPES = {"int8": (torch.int8,), "e4m3": (torch.float8_e4m3fn, torch.uint8)}


def _host_copy(t: torch.Tensor) -> torch.Tensor:
    # a private host copy: safetensors refuses tensors that share storage
    t = t.detach()
    return t.to("cpu").contiguous() if t.device.type != "cpu" else t.contiguous().clone()


def _meta_of(q: QuantizedTensor) -> dict:
    return {"original_shape": [int(d) for d in q.original_shape], "block_size": int(q.block_size),
            "code_format": q.code_format, "code_layout": q.code_layout, "outlier_tile_max": int(q.outlier_tile_max)}


def save_quantized(tensors: Mapping[str, QuantizedTensor], path: str,
                   extra: Optional[Mapping[str, torch.Tensor]] = None) -> None:
    """Write the QuantizedTensors of ``tensors`` (and the plain tensors of
    ``extra``) to the safetensors file ``path``.  Names may not contain '/'."""
    flat: Dict[str, torch.Tensor] = {}
    entries = {}
    for name, q in tensors.items():
        if "/" in name or not isinstance(q, QuantizedTensor):
            raise ValueError(f"save_quantized: bad entry {name!r} ({type(q).__name__})")
        entries[name] = _meta_of(q)
        for f in _TENSOR_FIELDS:
            t = getattr(q, f)
            if t is not None:
                flat[f"{name}/{f}"] = _host_copy(t)
    for name, t in (extra or {}).items():
        if "/" in name or name in entries or not isinstance(t, torch.Tensor):
            raise ValueError(f"save_quantized: bad extra tensor {name!r}")
        flat[name] = _host_copy(t)
    meta = {"format": FORMAT_NAME, "version": str(FORMAT_VERSION), "entries": json.dumps(entries, sort_keys=True)}
    save_file(flat, path, metadata=meta)


def _check_entry(name: str, q: QuantizedTensor) -> None:
    """Size relations every QuantizedTensor of the two formats satisfies."""
    def bad(why):
        raise ValueError(f"load_quantized: entry {name!r}: {why}")
    if q.code_format not in _CODE_DTYPES:
        bad(f"unknown code_format {q.code_format!r}")
    if q.fp8_data.dtype not in _CODE_DTYPES[q.code_format]:
        bad(f"codes of dtype {q.fp8_data.dtype} for format {q.code_format}")
    numel = q.original_shape.numel()
    G = q.block_size
    if G < 1:
        bad(f"block_size {G}")
    nnz = q.outlier_indices.numel()
    if q.fp16_outliers.dtype != torch.float16 or q.fp16_outliers.numel() != nnz:
        bad("outlier values do not match the outlier indices")
    if q.outlier_indices.dtype != torch.int64 or q.scale_factors.dtype != torch.float16:
        bad("index or scale dtype")
    nblocks = (numel + G - 1) // G
    if q.scale_factors.numel() != nblocks:
        bad(f"{q.scale_factors.numel()} scales for {nblocks} blocks")
    ncodes = q.fp8_data.numel()
    if q.code_format == "int8" and ncodes != nblocks * G - nnz:
        bad(f"{ncodes} int8 codes, expected {nblocks * G - nnz}")
    if q.code_format == "e4m3" and ncodes not in (numel, nblocks * G):
        bad(f"{ncodes} e4m3 codes for {numel} elements")
    if q.code_layout not in ("flat", "tiled"):
        bad(f"code_layout {q.code_layout!r}")
    if q.code_layout == "tiled" and not tiled_eligible(q.original_shape, G):
        bad(f"tiled codes for shape {tuple(q.original_shape)} and block {G}")
    # The index lists drive device reads (the GEMV reads x at each outlier's
    # column, the dequantize kernel writes at each flat index): every value
    # is checked here, on the host, before the tensors reach a kernel.
    idx = q.outlier_indices
    if nnz and (int(idx[0]) < 0 or int(idx[-1]) >= nblocks * G or (nnz > 1 and not bool((idx[1:] > idx[:-1]).all()))):
        bad("outlier indices are not ascending inside the padded tensor")
    K = int(q.original_shape[-1]) if len(q.original_shape) else 1
    rows = numel // K if K else 0
    inside = int((idx < rows * K).sum()) if nnz else 0  # outliers in the padding have no row
    if q.outlier_row_ptr is not None:
        rp = q.outlier_row_ptr
        if rp.dtype != torch.int32 or rp.numel() != rows + 1:
            bad("row pointer dtype or length")
        if int(rp[0]) != 0 or int(rp[-1]) != inside or (rows and not bool((rp[1:] >= rp[:-1]).all())):
            bad("row pointer is not a CSR pointer over the outliers")
        if rows and not torch.equal(rp[1:].long() - rp[:-1].long(),
                                    torch.bincount(idx[:inside] // K, minlength=rows)):
            bad("row pointer does not match the outlier indices")
    if q.outlier_cols is not None:
        if q.outlier_cols.dtype != torch.int32 or q.outlier_cols.numel() != nnz:
            bad("outlier column dtype or count")
        if not torch.equal(q.outlier_cols[:inside].long(), idx[:inside] % K):
            bad("outlier columns do not match the outlier indices")
    if (q.outlier_tile_ptr is None) != (q.outlier_tile_ent is None):
        bad("block list pointer and entries must come together")
    if q.outlier_tile_ptr is not None:
        if q.outlier_row_ptr is None or q.outlier_cols is None or not tiles_eligible(q.original_shape):
            bad("block lists without CSR lists or for a shape without 16 x 64 blocks")
        tp, te = q.outlier_tile_ptr, q.outlier_tile_ent
        if tp.dtype != torch.int32 or te.dtype != torch.int32:
            bad("block list dtype")
        exp_ptr, exp_ent = _block_lists(idx[:inside], q.fp16_outliers[:inside], rows, K)
        if not torch.equal(tp, exp_ptr) or te.numel() != inside + 64 or not torch.equal(te[:inside], exp_ent):
            bad("block lists do not match the outliers")
        if int(q.outlier_tile_max) != (int((tp[1:] - tp[:-1]).max()) if inside else 0):
            bad(f"outlier_tile_max {q.outlier_tile_max} does not match the block lists")


def _block_lists(idx: torch.Tensor, vals: torch.Tensor, N: int, K: int):
    """The 16 x 64 block lists of aq_outlier_tiles, rebuilt on the host:
    entry (fp16 value << 16) | r << 6 | k, ordered by block, row, column."""
    n, c = idx // K, idx % K
    blk = (n // 16) * (K // 64) + c // 64
    ent = (vals.view(torch.int16).to(torch.int64) & 0xFFFF) << 16 | (n % 16) << 6 | (c % 64)
    order = torch.sort(blk, stable=True).indices
    ptr = torch.searchsorted(blk[order], torch.arange((N // 16) * (K // 64) + 1, dtype=torch.int64))
    ent = ent[order]
    return ptr.to(torch.int32), torch.where(ent >= 1 << 31, ent - (1 << 32), ent).to(torch.int32)


def load_quantized(path: str, device="cpu") -> Tuple[Dict[str, QuantizedTensor], Dict[str, torch.Tensor]]:
    """Read a file written by ``save_quantized``: (quantized tensors, plain
    tensors), every tensor on ``device``."""
    dev = torch.device(device)
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT_NAME:
            raise ValueError(f"load_quantized: {path} is not an {FORMAT_NAME} file")
        if meta.get("version") != str(FORMAT_VERSION):
            raise ValueError(f"load_quantized: unsupported version {meta.get('version')!r} (this build reads "
                             f"{FORMAT_VERSION})")
        try:
            entries = json.loads(meta["entries"])
        except (KeyError, ValueError) as e:
            raise ValueError(f"load_quantized: unreadable entry table in {path}") from e
        keys = set(f.keys())
        out: Dict[str, QuantizedTensor] = {}
        used = set()
        for name, m in entries.items():
            fields = {}
            for fld in _TENSOR_FIELDS:
                k = f"{name}/{fld}"
                if k in keys:
                    fields[fld] = f.get_tensor(k)
                    used.add(k)
                elif fld in _REQUIRED:
                    raise ValueError(f"load_quantized: entry {name!r} lacks {fld}")
                else:
                    fields[fld] = None
            try:
                q = QuantizedTensor(original_shape=torch.Size(m["original_shape"]), block_size=int(m["block_size"]),
                                    code_format=m["code_format"], code_layout=m["code_layout"],
                                    outlier_tile_max=int(m["outlier_tile_max"]), **fields)
            except (KeyError, TypeError) as e:
                raise ValueError(f"load_quantized: entry {name!r} has incomplete metadata") from e
            _check_entry(name, q)
            out[name] = q
        extra = {k: f.get_tensor(k) for k in sorted(keys - used) if "/" not in k}
        stray = sorted(k for k in keys - used if "/" in k)
        if stray:
            raise ValueError(f"load_quantized: tensors without an entry: {stray[:4]}")
    if dev.type != "cpu":
        out = {k: q.to(dev) for k, q in out.items()}
        extra = {k: t.to(dev) for k, t in extra.items()}
    return out, extra


def _quantized_linears(model: nn.Module):
    return [(n, m) for n, m in model.named_modules() if type(m).__name__ == "QuantizedLinear"]


def save_quantized_model(model: nn.Module, path: str) -> int:
    """Store every QuantizedLinear of ``model`` (weights and bias) under its
    module name.  Returns the number of layers written."""
    qls = _quantized_linears(model)
    tensors, extra = {}, {}
    for name, m in qls:
        key = name.replace("/", "_")
        tensors[key] = m.quantized_weights
        if m.bias is not None:
            extra[f"{key}.bias"] = m.bias
    save_quantized(tensors, path, extra)
    return len(qls)


def load_quantized_model(model: nn.Module, path: str, device=None) -> int:
    """Swap the Linear modules of ``model`` named in ``path`` for
    QuantizedLinear modules holding the stored weights; the model is cast to
    fp16 first, as apply_atlas_quantization_to_model does.  Every named
    module must exist and be an nn.Linear (or QuantizedLinear) of the stored
    shape, else ValueError is raised before anything is replaced.  Returns
    the number of modules replaced."""
    from ..integration.atlas_wrappers import QuantizedLinear
    from ..integration.model_modifier import _replace_module

    dev = torch.device(device) if device is not None else torch.device("cpu")
    weights, extra = load_quantized(path, dev)
    plan = []
    for name, q in weights.items():
        try:
            mod = model.get_submodule(name)
        except AttributeError:
            raise ValueError(f"load_quantized_model: the model has no module {name!r}") from None
        if isinstance(mod, nn.Linear):
            shape = (mod.out_features, mod.in_features)
        elif type(mod).__name__ == "QuantizedLinear":
            shape = tuple(mod.original_shape)
        else:
            raise ValueError(f"load_quantized_model: {name!r} is a {type(mod).__name__}, not a Linear")
        if tuple(q.original_shape) != shape:
            raise ValueError(f"load_quantized_model: {name!r} has shape {shape}, stored {tuple(q.original_shape)}")
        bias = extra.get(f"{name}.bias")
        if isinstance(mod, nn.Linear) and (mod.bias is None) != (bias is None):
            raise ValueError(f"load_quantized_model: bias presence of {name!r} differs from the file")
        plan.append((name, q, bias))
    try:
        model.to(dtype=torch.float16)
    except Exception as e:  # same tolerance as apply_atlas_quantization_to_model
        print(f"Warning: cast to fp16 failed: {e}")
    for name, q, bias in plan:
        parent_name, child = name.rsplit(".", 1) if "." in name else ("", name)
        parent = model.get_submodule(parent_name) if parent_name else model
        _replace_module(parent, child, QuantizedLinear(q, bias))
    return len(plan)
