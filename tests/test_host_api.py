"""Host-side logic of the reference API mirror that needs no GPU: type checks,
empty tensors, the QuantizedTensor container, module discovery, and that the
compute path refuses to run without a HIP device instead of falling back."""
import pytest
import torch
import torch.nn as nn

from atlasinfer_core.quant import adaptive_quantizer as AQ
from integration import atlas_wrappers as AW
from integration import model_modifier as MM


def test_import_aliases_are_the_implementation():
    import atlasinfer_amd.quant.adaptive_quantizer as impl
    import atlasinfer_amd.integration.atlas_wrappers as w
    import atlasinfer_amd.integration.model_modifier as m
    assert AQ is impl and AW is w and MM is m


def test_non_tensor_input_raises_type_error():
    with pytest.raises(TypeError):
        AQ.quantize_tensor([1.0, 2.0])


def test_empty_tensor_round_trip_shape():
    e = torch.empty((0, 10), dtype=torch.float16)
    for fmt in ["int8", "e4m3"]:
        q = AQ.quantize_tensor(e, code_format=fmt)
        assert q.original_shape == e.shape and q.fp8_data.numel() == 0
        AQ.clear_dequantized_cache()
        assert AQ.dequantize_tensor(q, torch.device("cpu")).shape == e.shape


def test_bad_format_and_block_size():
    t = torch.ones(4, 4, dtype=torch.float16)
    with pytest.raises(ValueError):
        AQ.quantize_tensor(t, code_format="int4")
    with pytest.raises(ValueError):
        AQ.quantize_tensor(t, block_size=0)


def test_quantized_tensor_fields_and_footprint():
    q = AQ.QuantizedTensor(torch.zeros(10, dtype=torch.int8), torch.zeros(2, dtype=torch.float16),
                           torch.zeros(2, dtype=torch.long), torch.zeros(1, dtype=torch.float16),
                           torch.Size([3, 4]), 64)
    assert q._fields[:6] == ("fp8_data", "fp16_outliers", "outlier_indices", "scale_factors", "original_shape",
                             "block_size")
    assert q.code_format == "int8"  # a tuple built from the six reference fields keeps reference semantics
    assert q.memory_footprint(include_overhead=False) == 10 + 4 + 16 + 2
    assert q.memory_footprint() == 32 + 128
    assert q.to("cpu") is q


def test_compute_without_device_raises():
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    from atlasinfer_amd._lib import AQError
    with pytest.raises(AQError):
        AQ.quantize_tensor(torch.ones(4, 128, dtype=torch.float16))
    with pytest.raises(RuntimeError):
        AW.QuantizedLinear(AQ.quantize_tensor(torch.empty(0, 4, dtype=torch.float16)), None)(
            torch.ones(1, 4, dtype=torch.float16))


class Tiny(nn.Module):
    def __init__(self):
        super().__init__()
        self.block = nn.Sequential(nn.Linear(8, 8), nn.ReLU(), nn.Linear(8, 4))
        self.lm_head = nn.Linear(4, 4)
        self.embed_tokens = nn.Embedding(3, 8)


def test_find_modules_and_exclusions():
    m = Tiny()
    names = [n for n, _ in MM.find_modules(m, [nn.Linear], exclude_names=["lm_head", "embed_tokens"])]
    assert names == ["block.0", "block.2"]
    names = [n for n, _ in MM.find_modules(m, [], target_names=["Embedding"])]
    assert names == ["embed_tokens"]
    assert set(MM.MODEL_LAYER_PATTERNS) == {"opt", "llama", "mistral", "gemma"}
    assert MM._get_model_patterns("bert") is None


def test_extra_repr_format():
    q = AQ.quantize_tensor(torch.empty(0, 4, dtype=torch.float16))
    r = AW.QuantizedLinear(q, None).extra_repr()
    assert r.startswith("quantized_shape=torch.Size([0, 4]), bias=False, device=")


def test_device_int_reads_once_and_acts_as_int():
    """quantize_tensor hands back the block lists' largest count as a
    DeviceInt (read from its one-element tensor when first used): it
    compares, adds, converts for ctypes, copies and pickles like the int it
    holds, and reads the tensor only once."""
    import copy
    import ctypes
    import pickle
    from atlasinfer_amd.quant.adaptive_quantizer import DeviceInt
    t = torch.tensor(70, dtype=torch.int32)
    d = DeviceInt(t)
    assert d > 64 and d >= 70 and d == 70 and not d < 70 and d <= 70
    assert d - 1 == 69 and 1 + d == 71 and int(d) == 70 and hash(d) == hash(70)
    t.fill_(3)  # already read: later changes to the tensor do not matter
    assert int(d) == 70
    assert (ctypes.c_int64 * 1)(DeviceInt(torch.tensor(9)))[0] == 9
    assert int(copy.deepcopy(DeviceInt(torch.tensor(5)))) == 5
    assert int(pickle.loads(pickle.dumps(DeviceInt(torch.tensor(6))))) == 6
    # a stored count of 0 is falsy, like the int (a tensor object is always truthy)
    assert not DeviceInt(torch.tensor(0)) and bool(DeviceInt(torch.tensor(2)))
    assert DeviceInt(torch.tensor(3)) != 4 and not DeviceInt(torch.tensor(3)) != 3
    assert DeviceInt(torch.tensor(3)) * 2 == 6 and 2 * DeviceInt(torch.tensor(3)) == 6


def test_dequant_cache_never_serves_another_objects_weights():
    """The dequant cache is keyed by id(QuantizedTensor), as in the
    reference (adaptive_quantizer.py:153-171,248-249), but an id is only a
    hit for the very object it was stored for: (a) each entry keeps its
    QuantizedTensor alive, so while it exists the id cannot be handed to a
    new object; (b) an entry found under an object's id but stored for
    another object is recomputed, not returned."""
    import gc

    def empty_qt(cols):
        return AQ.quantize_tensor(torch.empty(0, cols, dtype=torch.float16))

    AQ.clear_dequantized_cache()
    q = empty_qt(4)
    w = AQ.dequantize_tensor(q, torch.device("cpu"))
    assert AQ.dequantize_tensor(q, torch.device("cpu")) is w  # memoised by identity
    qid = id(q)
    del q
    gc.collect()
    # still alive in its cache entry, so id(q) stays taken
    assert id(AQ._dequantized_weights_cache[qid][0]) == qid
    AQ.clear_dequantized_cache(qid)
    assert qid not in AQ._dequantized_weights_cache
    # a stale entry under a live object's id (what id reuse would produce)
    q2 = empty_qt(8)
    impostor = torch.full((0, 4), 1.0, dtype=torch.float16)
    AQ._dequantized_weights_cache[id(q2)] = (empty_qt(4), impostor)
    out = AQ.dequantize_tensor(q2, torch.device("cpu"))
    assert out is not impostor and out.shape == (0, 8)
    assert AQ._dequantized_weights_cache[id(q2)][0] is q2
    AQ.clear_dequantized_cache()
