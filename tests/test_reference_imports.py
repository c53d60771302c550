"""Every name the reference's own modules, example and tests import from the
reference's packages resolves here, to this implementation, with the repo
root on the path (as the reference's callers put theirs).  The lists are
written out from the reference files cited on each entry, so a missing
module or name fails here by name."""
import importlib

import pytest
import torch
import torch.nn as nn

# (module path, names, where the reference imports them)
REFERENCE_IMPORTS = [
    ("atlasinfer_core.memory.unified_memory_manager", ["UnifiedMemoryManager"],
     "examples/run_atlas_inference.py:16, integration/model_modifier.py:12, tests/test_memory_manager.py:9"),
    ("atlasinfer_core.utils.helpers", ["estimate_quantized_model_vram", "cleanup_memory"],
     "examples/run_atlas_inference.py:17"),
    ("atlasinfer_core.utils.helpers", ["cleanup_memory"],
     "integration/model_modifier.py:13, tests/test_memory_manager.py:11"),
    ("atlasinfer_core.utils.helpers", ["map_structure"], "atlasinfer_core/utils/weight_offloader.py:6"),
    ("integration.model_modifier",
     ["apply_atlas_quantization_to_model", "apply_atlas_attention_wrapper", "setup_offloading_hooks",
      "_get_model_patterns"], "examples/run_atlas_inference.py:19-24"),
    ("integration.atlas_wrappers", ["QuantizedLinear", "AtlasAttentionWrapper"],
     "integration/model_modifier.py:10"),
    ("atlasinfer_core.quant.adaptive_quantizer", ["QuantizedTensor", "quantize_tensor"],
     "integration/model_modifier.py:11, atlasinfer_core/utils/weight_offloader.py:20"),
    ("atlasinfer_core.utils.weight_offloader", ["QuantizedTensorOffloadHook"], "integration/model_modifier.py:15"),
    ("atlasinfer_core.quant.adaptive_quantizer", ["dequantize_tensor", "clear_dequantized_cache"],
     "integration/atlas_wrappers.py:17"),
    ("atlasinfer_core.quant.adaptive_quantizer",
     ["quantize_tensor", "dequantize_tensor", "QuantizedTensor", "clear_dequantized_cache"],
     "tests/test_quantizer.py:5"),
    # names the reference's modules define and its callers reach as attributes
    ("integration.model_modifier", ["find_modules", "_replace_module", "MODEL_LAYER_PATTERNS"],
     "integration/model_modifier.py:21-92"),
    ("atlasinfer_core.quant.adaptive_quantizer", ["calculate_zscore_manual"], "adaptive_quantizer.py:44"),
    ("atlasinfer_core.utils.weight_offloader", ["_clear_specific_dequant_cache", "clear_all_dequant_cache",
                                                "map_structure"], "atlasinfer_core/utils/weight_offloader.py:6,28,36"),
]


@pytest.mark.parametrize("module,names,where", REFERENCE_IMPORTS, ids=[f"{m}:{','.join(n)}" for m, n, _ in
                                                                        REFERENCE_IMPORTS])
def test_reference_import_resolves(module, names, where):
    mod = importlib.import_module(module)
    missing = [n for n in names if not hasattr(mod, n)]
    assert not missing, f"{module} lacks {missing} (imported at reference {where})"
    assert mod.__name__.startswith("atlasinfer_amd."), f"{module} is not an alias of the implementation"


def test_helpers_alias_is_the_implementation():
    import atlasinfer_core.utils.helpers as ref_path
    import atlasinfer_amd.utils.helpers as impl
    from atlasinfer_core.utils import weight_offloader as wo
    assert ref_path is impl and wo.map_structure is impl.map_structure


def test_map_structure_shapes():
    from atlasinfer_core.utils.helpers import map_structure
    from atlasinfer_core.quant.adaptive_quantizer import QuantizedTensor
    from collections import OrderedDict, namedtuple
    seen = []

    def f(o):
        seen.append(type(o).__name__)
        return ("mapped", o) if isinstance(o, QuantizedTensor) else o + 1

    qt = QuantizedTensor(torch.zeros(4, dtype=torch.int8), torch.zeros(0, dtype=torch.float16),
                         torch.zeros(0, dtype=torch.long), torch.ones(1, dtype=torch.float16), torch.Size([2, 2]), 4)
    P = namedtuple("P", "a b")
    obj = OrderedDict(x=torch.zeros(2), y=[torch.zeros(1), (torch.ones(1), 7)], z=P(torch.zeros(1), "s"), q=qt,
                      n=None)
    out = map_structure(f, obj)
    assert type(out) is dict and list(out) == ["x", "y", "z", "q", "n"]
    assert torch.equal(out["x"], torch.ones(2))
    assert isinstance(out["y"], list) and isinstance(out["y"][1], tuple) and out["y"][1][1] == 7
    assert torch.equal(out["y"][1][0], torch.full((1,), 2.0))
    assert type(out["z"]) is P and out["z"].b == "s" and torch.equal(out["z"].a, torch.ones(1))
    assert out["q"][0] == "mapped" and out["q"][1] is qt  # handed over whole
    assert out["n"] is None
    assert seen.count("QuantizedTensor") == 1


class _TiedLM(nn.Module):
    def __init__(self):
        super().__init__()
        self.embed_tokens = nn.Embedding(10, 16)
        self.norm = nn.LayerNorm(16)
        self.fc1 = nn.Linear(16, 32)
        self.fc2 = nn.Linear(32, 16, bias=False)
        self.lm_head = nn.Linear(16, 10, bias=False)
        self.lm_head.weight = self.embed_tokens.weight  # tied


def _param_bytes(ps):
    return sum(p.element_size() * p.nelement() for p in ps)


def test_estimate_vram_plain_model_counts_each_parameter_once():
    from atlasinfer_core.utils.helpers import estimate_quantized_model_vram
    m = _TiedLM().half()
    uniq = {id(p): p for p in m.parameters()}.values()
    assert estimate_quantized_model_vram(m) == _param_bytes(uniq)


def test_estimate_vram_after_swap():
    """After the swap, each QuantizedLinear counts its QuantizedTensor's
    components and its bias; the rest count their parameters.  Two layers
    sharing one QuantizedTensor count it once."""
    from atlasinfer_core.utils.helpers import estimate_quantized_model_vram
    from atlasinfer_core.quant.adaptive_quantizer import QuantizedTensor
    from integration.atlas_wrappers import QuantizedLinear
    m = _TiedLM().half()

    def qt_of(n, k):
        return QuantizedTensor(torch.zeros(n * k, dtype=torch.uint8), torch.zeros(3, dtype=torch.float16),
                               torch.zeros(3, dtype=torch.long), torch.zeros(n, dtype=torch.float16),
                               torch.Size([n, k]), k, "e4m3", torch.zeros(n + 1, dtype=torch.int32),
                               torch.zeros(3, dtype=torch.int32))

    q1, q2 = qt_of(32, 16), qt_of(16, 32)
    m.fc1 = QuantizedLinear(q1, m.fc1.bias.detach().clone())
    m.fc2 = QuantizedLinear(q2, None)
    m.extra = QuantizedLinear(q2, None)  # shares fc2's weight object
    plain = [m.embed_tokens.weight, m.norm.weight, m.norm.bias]
    want = (_param_bytes(plain) + q1.memory_footprint(include_overhead=False) + 32 * 2
            + q2.memory_footprint(include_overhead=False))
    assert estimate_quantized_model_vram(m) == want
    # include_overhead=False: the 128-byte allowance is not counted
    assert q1.memory_footprint() - q1.memory_footprint(include_overhead=False) == 128


def test_cleanup_memory_runs_without_device(capsys):
    from atlasinfer_core.utils.helpers import cleanup_memory
    cleanup_memory()
    out = capsys.readouterr().out
    assert "cleanup" in out
