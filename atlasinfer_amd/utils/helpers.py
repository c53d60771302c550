"""Small utilities the reference keeps in atlasinfer_core/utils/helpers.py
(importable under that path too):

* ``map_structure`` (reference helpers.py:9-45) -- apply a function to every
  tensor or QuantizedTensor inside nested dicts, lists and tuples;
* ``estimate_quantized_model_vram`` (reference :54-82) -- device bytes of a
  model's weights once its quantized layers are in place;
* ``cleanup_memory`` (reference :85-91) -- garbage collection and release of
  the device allocator's cached blocks.
"""
from __future__ import annotations

import gc
from collections.abc import Mapping
from typing import Any, Callable

import torch
import torch.nn as nn


def _is_quantized_tensor(obj: Any) -> bool:
    # matched by class name, as the reference's consumers do, so that a
    # QuantizedTensor imported under either package path is recognised
    return type(obj).__name__ == "QuantizedTensor"


def map_structure(func: Callable, obj: Any):
    """``func`` applied to every tensor and QuantizedTensor in ``obj``.

    Mappings come back as plain dicts, named tuples as the same named tuple
    type (a plain list when the type cannot be rebuilt from its elements),
    other lists and tuples as their own type; anything else is returned as it
    is.  A QuantizedTensor is handed to ``func`` whole, not field by field,
    which is what the reference's QuantizedTensor branch (helpers.py:35-41)
    is written for; there it sits after the tuple branch, so the named tuple
    was rebuilt from its fields mapped one by one instead (the same result
    for a function that moves tensors, which is how the offload hook uses
    it)."""
    if _is_quantized_tensor(obj) or isinstance(obj, torch.Tensor):
        return func(obj)
    if isinstance(obj, Mapping):
        return {k: map_structure(func, v) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        items = [map_structure(func, o) for o in obj]
        if isinstance(getattr(obj, "_fields", None), tuple):
            try:
                return type(obj)(*items)
            except TypeError:
                return items
        return type(obj)(items)
    return obj


def _tensor_bytes(t: torch.Tensor) -> int:
    return t.element_size() * t.nelement()


def estimate_quantized_model_vram(model: nn.Module) -> int:
    """Bytes the model's weights take on a device (activations and KV cache
    not included; reference helpers.py:54-82).

    A ``QuantizedLinear`` counts its QuantizedTensor's component tensors
    (``memory_footprint(include_overhead=False)``) and its bias; every other
    module counts its own parameters.  A tensor, QuantizedTensor or parameter
    reachable from several modules (tied embeddings, shared weights) counts
    once."""
    seen = set()
    total = 0

    def add(obj: Any, nbytes: Callable[[], int]) -> None:
        nonlocal total
        if obj is None or id(obj) in seen:
            return
        seen.add(id(obj))
        total += nbytes()

    for module in model.modules():
        if type(module).__name__ == "QuantizedLinear":
            qt = getattr(module, "quantized_weights", None)
            if qt is not None and hasattr(qt, "memory_footprint"):
                add(qt, lambda: int(qt.memory_footprint(include_overhead=False)))
            bias = getattr(module, "bias", None)
            if isinstance(bias, torch.Tensor):
                add(bias, lambda: _tensor_bytes(bias))
            continue
        for p in module.parameters(recurse=False):
            add(p, lambda: _tensor_bytes(p))
    return total


def cleanup_memory() -> None:
    """Collect garbage, then return the device allocator's unused cached
    blocks to the driver (reference helpers.py:85-91)."""
    print("Running memory cleanup...")
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    print("Memory cleanup done.")
