"""Swap a model's nn.Linear layers for QuantizedLinear.

Mirrors the quantization half of /root/reference/integration/model_modifier.py
(``MODEL_LAYER_PATTERNS`` :21-50, ``_get_model_patterns`` :52-56,
``_replace_module`` :58-76, ``find_modules`` :78-92,
``apply_atlas_quantization_to_model`` :95-143); also importable as
``integration.model_modifier``.  Differences: the weights are quantized on the
GPU (bit-identical to a CPU run of the same algorithm) and stay there, and
this module has no import-time dependency on the KV-cache tier (lmdb).
"""
from __future__ import annotations

import gc
import traceback
from typing import Dict, List, Optional, Tuple, Type

import torch
import torch.nn as nn

from .. import _lib
from ..quant.adaptive_quantizer import quantize_tensor, quantize_tensors
from .atlas_wrappers import QuantizedLinear

MODEL_LAYER_PATTERNS = {
    "opt": {
        "linear_types": [nn.Linear],
        "attention_type": ["OPTAttention", "OPTSdpaAttention"],
        "decoder_layer_type": "OPTDecoderLayer",
        "decoder_block_path": "model.decoder.layers",
        "attention_subpath": "self_attn",
    },
    "llama": {
        "linear_types": [nn.Linear],
        "attention_type": ["LlamaAttention", "LlamaSdpaAttention"],
        "decoder_layer_type": "LlamaDecoderLayer",
        "decoder_block_path": "model.layers",
        "attention_subpath": "self_attn",
    },
    "mistral": {
        "linear_types": [nn.Linear],
        "attention_type": ["MistralAttention", "MistralSdpaAttention"],
        "decoder_layer_type": "MistralDecoderLayer",
        "decoder_block_path": "model.layers",
        "attention_subpath": "self_attn",
    },
    "gemma": {
        "linear_types": [nn.Linear],
        "attention_type": ["GemmaAttention", "GemmaSdpaAttention"],
        "decoder_layer_type": "GemmaDecoderLayer",
        "decoder_block_path": "model.layers",
        "attention_subpath": "self_attn",
    },
}


def _get_model_patterns(model_type: str) -> Optional[Dict]:
    patterns = MODEL_LAYER_PATTERNS.get(model_type)
    if patterns is None:
        print(f"Warning: No layer patterns for '{model_type}'.")
    return patterns


def _replace_module(parent_module: nn.Module, child_name: str, new_module: nn.Module):
    """setattr the new module in place of the old one."""
    setattr(parent_module, child_name, new_module)


def find_modules(model: nn.Module, target_types: List[Type], target_names: List[str] = [],
                 exclude_names: List[str] = []) -> List[Tuple[str, nn.Module]]:
    """Modules matching a type (isinstance) or a class name, skipping any whose
    qualified name contains an excluded substring (reference :78-92)."""
    found = []
    if not isinstance(target_names, list):
        target_names = [target_names] if target_names else []
    if not isinstance(target_types, list):
        target_types = [target_types] if target_types else []
    if not isinstance(exclude_names, list):
        exclude_names = [exclude_names] if exclude_names else []
    for name, module in model.named_modules():
        if any(ex and ex in name for ex in exclude_names):
            continue
        type_match = any(isinstance(module, t) for t in target_types if t is not None)
        name_match = type(module).__name__ in target_names
        if type_match or name_match:
            found.append((name, module))
    return found


def apply_atlas_quantization_to_model(model: nn.Module, model_type: str, quantization_config: Dict,
                                      excluded_layers: List[str] = ["lm_head", "embed_tokens", "embeddings"],
                                      *, device: Optional[torch.device] = None, fuse_siblings: bool = False):
    """Quantize every non-excluded nn.Linear of ``model`` in place
    (reference :95-143).  ``quantization_config`` is splatted into
    quantize_tensor (block_size, z_threshold, code_format).  Returns
    (layers_replaced, layers_failed).  ``fuse_siblings`` (not in the
    reference) links q/k/v and gate/up projections of one parent into a
    SiblingGroup (see link_sibling_linears)."""
    print(f"\n--- Applying Atlas Quantization ({model_type}) ---")
    patterns = _get_model_patterns(model_type)
    if patterns is None:
        print("ERROR: No patterns.")
        return
    dev = _lib.compute_device(torch.device(device) if device is not None else None)
    try:
        model.to(dtype=torch.float16)
    except Exception as e:  # same tolerance as the reference's pre-quant move
        print(f"Warning: Pre-quant cast failed: {e}")
    target_linear_types = patterns.get("linear_types", [])
    if not target_linear_types:
        print("Warning: No linear types.")
        return
    linear_modules = find_modules(model, target_types=target_linear_types, exclude_names=excluded_layers)
    if not linear_modules:
        print("Warning: No linear layers found.")
        return
    print(f"Found {len(linear_modules)} linear layers to quantize...")
    replaced, failed = 0, 0
    # Linears are quantized in runs of up to 8 (quantize_tensors: one launch
    # for the members sharing a block size, the same results as one call
    # each); a run that fails is retried member by member, so each failure
    # is reported and skipped on its own as the reference's loop does
    pending = []  # (parent, child name, name, fp16 weight, bias)

    def flush():
        nonlocal replaced, failed
        if not pending:
            return
        try:
            qts = quantize_tensors([p[3] for p in pending], **quantization_config)
        except Exception:
            qts = [None] * len(pending)
        for (parent, child, name, w, b), qt in zip(pending, qts):
            try:
                if qt is None:
                    qt = quantize_tensor(w, **quantization_config)
                _replace_module(parent, child, QuantizedLinear(qt, b))
                replaced += 1
            except Exception as e:
                print(f"!! FAILED quant layer {name}: {e}")
                traceback.print_exc()
                failed += 1
        pending.clear()

    for name, module in list(linear_modules):
        parent_name, child_name = name.rsplit(".", 1) if "." in name else ("", name)
        parent = model.get_submodule(parent_name) if parent_name else model
        if type(getattr(parent, child_name, None)).__name__ == "QuantizedLinear":
            continue
        try:
            if not hasattr(module, "weight") or module.weight is None:
                print(f"Warn: No weight {name}. Skip.")
                failed += 1
                continue
            w = module.weight.data.to(dtype=torch.float16, device=dev)
            b = module.bias.data.to(dtype=torch.float16, device=dev).clone() if getattr(module, "bias", None) is not None else None
            pending.append((parent, child_name, name, w, b))
            del w, module
        except Exception as e:
            print(f"!! FAILED quant layer {name}: {e}")
            traceback.print_exc()
            failed += 1
        if len(pending) == 8:
            flush()
    flush()
    gc.collect()
    if fuse_siblings:
        print(f"Linked {link_sibling_linears(model)} sibling groups for grouped decode launches")
    print(f"--- Quantization complete. Replaced: {replaced}, Failed/Skipped: {failed} ---")
    return replaced, failed


SIBLING_NAMES = (("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj"))


def link_sibling_linears(model: nn.Module, names=SIBLING_NAMES) -> int:
    """Link the QuantizedLinear children of one parent that a forward calls
    in turn on the same input (``names``, first member first) into a
    SiblingGroup: at decode sizes the first one's forward runs one grouped
    launch and the others take their outputs.  Members must share
    in_features and code format.  Returns the number of groups linked."""
    from .atlas_wrappers import SiblingGroup
    n = 0
    for parent in model.modules():
        for group in names:
            mods = [getattr(parent, c, None) for c in group]
            if not all(type(m).__name__ == "QuantizedLinear" for m in mods):
                continue
            qs = [m.quantized_weights for m in mods]
            if len({int(q.original_shape[-1]) for q in qs}) != 1 or len({q.code_format for q in qs}) != 1:
                continue
            g = SiblingGroup(mods)
            for m in mods:
                m._group = g
            n += 1
    return n


FINAL_NORM_PATHS = ("model.decoder.final_layer_norm", "model.norm", "decoder.norm")


def _shares_parameters(module: nn.Module, model: nn.Module) -> bool:
    """Whether a parameter of ``module`` also belongs to a module outside it
    (a tied lm_head / embedding weight)."""
    own = {id(p) for p in module.parameters()}
    inside = {id(m) for m in module.modules()}
    for m in model.modules():
        if id(m) in inside:
            continue
        if any(id(p) in own for p in m.parameters(recurse=False)):
            return True
    return False


def setup_offloading_hooks(model: nn.Module, model_type: str, gpu_device: torch.device, prefetch_depth: int = 1):
    """Stream the weights of the decoder blocks, the final norm and the
    lm_head from pinned host memory (reference :211-268, which attaches
    QuantizedTensorOffloadHook with offload=True to the same modules).

    Every hooked module's parameters, buffers and QuantizedLinear weights
    move to pinned host memory now; in a forward, each module's weights are
    on ``gpu_device`` only for its own forward, and the next
    ``prefetch_depth`` modules (in forward order, the first blocks again
    after the lm_head) are copied on a side stream meanwhile (0: each
    module's copy is issued at its own forward).  Unlike the reference, the
    final norm is hooked whatever its type and the lm_head whatever its type
    unless its weight is tied to a module outside it (that one stays where
    it is).  Modules that are not hooked (embeddings, rotary tables) stay
    where they are.  Returns the WeightStreamer (its ``stats`` count the
    prefetched and on-demand copies and the bytes copied)."""
    from accelerate.hooks import add_hook_to_module

    from ..utils.weight_offloader import QuantizedTensorOffloadHook, WeightStreamer

    print("\n--- Setting up weight streaming hooks ---")
    patterns = _get_model_patterns(model_type)
    if patterns is None:
        print("ERROR: No patterns.")
        return None
    path = patterns.get("decoder_block_path")
    try:
        blocks = model.get_submodule(path)
    except AttributeError:
        print(f"Warn: decoder block path '{path}' not found.")
        return None
    if not isinstance(blocks, nn.ModuleList):
        print("Warn: decoder blocks are not an nn.ModuleList.")
        return None
    streamer = WeightStreamer(gpu_device, depth=prefetch_depth)
    hooked = list(blocks)
    for p in FINAL_NORM_PATHS:
        try:
            hooked.append(model.get_submodule(p))
            break
        except AttributeError:
            continue
    lm_head = getattr(model, "lm_head", None)
    if lm_head is not None:
        if _shares_parameters(lm_head, model):
            print("lm_head shares its weight with another module: left in place.")
        else:
            hooked.append(lm_head)
    for m in hooked:
        streamer.register(m)
        add_hook_to_module(m, QuantizedTensorOffloadHook(execution_device=streamer.device, offload=True,
                                                         streamer=streamer))
    print(f"--- Streaming {len(hooked)} modules ({streamer.host_bytes() / 2**20:.1f} MiB pinned), "
          f"prefetch depth {prefetch_depth} ---")
    return streamer


def apply_atlas_attention_wrapper(model: nn.Module, model_type: str, memory_manager) -> Tuple[int, int]:
    """Wrap every decoder layer's attention (the pattern's attention class
    names) in an AtlasAttentionWrapper bound to ``memory_manager``, in place
    (reference :146-208).  Returns (wrapped, failed)."""
    from .atlas_wrappers import AtlasAttentionWrapper

    print(f"\n--- Applying Atlas Attention Wrapper ({model_type}) ---")
    patterns = _get_model_patterns(model_type)
    if patterns is None:
        print("ERROR: No patterns.")
        return 0, 0
    names = patterns.get("attention_type", [])
    names = names if isinstance(names, list) else [names]
    path, sub = patterns.get("decoder_block_path"), patterns.get("attention_subpath")
    try:
        layers = model.get_submodule(path)
    except AttributeError:
        print(f"Warn: Path not found: {path}")
        return 0, 0
    wrapped, failed = 0, 0
    for idx, layer in enumerate(layers):
        chain = sub.split(".")
        parent = layer.get_submodule(".".join(chain[:-1])) if len(chain) > 1 else layer
        attn = getattr(parent, chain[-1], None)
        if isinstance(attn, AtlasAttentionWrapper):
            print(f"Skipping wrapped layer {idx}.")
            continue
        if attn is None or type(attn).__name__ not in names:
            print(f"Warn: Type {type(attn).__name__} layer {idx} not target. Skip.")
            failed += 1
            continue
        q, k, v = (getattr(attn, n, None) for n in ("q_proj", "k_proj", "v_proj"))
        o = getattr(attn, "o_proj", None) or getattr(attn, "out_proj", None)
        try:
            w = AtlasAttentionWrapper(q, k, v, o, parent_layer=layer, memory_manager=memory_manager,
                                      layer_idx=idx, model_type=model_type)
        except ValueError as e:
            print(f"!! FAILED WRAP layer {idx}: {e}")
            failed += 1
            continue
        _replace_module(parent, chain[-1], w)
        wrapped += 1
    print(f"--- Attention wrapping complete. Wrapped: {wrapped}, Failed/Skipped: {failed} ---")
    return wrapped, failed
