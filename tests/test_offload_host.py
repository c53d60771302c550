"""Host-side parts of weight streaming that need no GPU: the reference's
import paths and names, map_structure, the hook's moves to the CPU, its
init_hook, and tied-weight detection for the lm_head."""
import pytest
import torch
import torch.nn as nn
from accelerate.hooks import AlignDevicesHook, add_hook_to_module

import atlasinfer_amd.utils.weight_offloader as impl
from atlasinfer_core.quant import adaptive_quantizer as AQ
from atlasinfer_core.utils import weight_offloader as WO
from integration import model_modifier as MM


def _qt():
    return AQ.QuantizedTensor(torch.zeros(4, dtype=torch.int8), torch.zeros(0, dtype=torch.float16),
                              torch.zeros(0, dtype=torch.int64), torch.ones(1, dtype=torch.float16),
                              torch.Size([4]), 4)


def test_reference_names_and_paths():
    assert WO is impl
    assert issubclass(WO.QuantizedTensorOffloadHook, AlignDevicesHook)
    for name in ("QuantizedTensorOffloadHook", "_clear_specific_dequant_cache", "clear_all_dequant_cache",
                 "map_structure", "WeightStreamer"):
        assert hasattr(WO, name), name
    assert callable(MM.setup_offloading_hooks)


def test_map_structure_nested_and_quantized_tensor_whole():
    seen = []

    def f(o):
        seen.append(type(o).__name__)
        return ("mapped", o) if isinstance(o, AQ.QuantizedTensor) else o + 1

    t = torch.zeros(2)
    q = _qt()
    out = WO.map_structure(f, {"a": [t, (t, 3)], "b": q, "c": "s", "d": None})
    assert torch.equal(out["a"][0], t + 1) and torch.equal(out["a"][1][0], t + 1) and out["a"][1][1] == 3
    assert isinstance(out["a"], list) and isinstance(out["a"][1], tuple)
    assert out["b"] == ("mapped", q) and out["c"] == "s" and out["d"] is None
    assert seen.count("QuantizedTensor") == 1  # handed over whole, not field by field


def test_move_to_device_on_cpu_targets():
    hook = WO.QuantizedTensorOffloadHook(execution_device=torch.device("cpu"), offload=True)
    cpu = torch.device("cpu")
    t = torch.ones(3)
    assert hook._move_to_device(t, cpu) is t
    assert hook._move_to_device(None, cpu) is None
    assert hook._move_to_device("x", cpu) == "x"
    q = _qt()
    assert hook._move_to_device(q, cpu) is q


def test_init_hook_keeps_parameters():
    """accelerate's offload set-up turns a module's own parameters into meta
    tensors; the hook here leaves them as they are (the streamer or
    module.to places them)."""
    ln = nn.LayerNorm(8)
    add_hook_to_module(ln, WO.QuantizedTensorOffloadHook(execution_device=torch.device("cpu"), offload=True))
    assert ln.weight.device.type == "cpu" and not ln.weight.is_meta
    y = ln(torch.randn(2, 8))
    assert y.shape == (2, 8)


def test_tied_lm_head_detected():
    emb = nn.Embedding(16, 8)
    head = nn.Linear(8, 16, bias=False)
    model = nn.Module()
    model.emb, model.lm_head = emb, head
    assert not MM._shares_parameters(head, model)
    head.weight = emb.weight
    assert MM._shares_parameters(head, model)


def test_streamer_needs_a_hip_device():
    with pytest.raises(ValueError):
        WO.WeightStreamer("cpu")
    with pytest.raises(ValueError):
        WO.WeightStreamer(torch.device("cuda", 0), depth=-1)


def test_discard_dequantized_only_drops_that_entry():
    AQ.clear_dequantized_cache()
    a, b = object(), object()
    with AQ._cache_lock:
        AQ._dequantized_weights_cache[id(a)] = (a, torch.zeros(1))
        AQ._dequantized_weights_cache[id(b)] = (b, torch.zeros(1))
    WO._clear_specific_dequant_cache(id(a))
    assert id(a) not in AQ._dequantized_weights_cache and id(b) in AQ._dequantized_weights_cache
    WO.clear_all_dequant_cache()
    assert len(AQ._dequantized_weights_cache) == 0
