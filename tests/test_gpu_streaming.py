"""Weight streaming (setup_offloading_hooks / QuantizedTensorOffloadHook):
a model whose decoder blocks, final norm and lm_head stream their weights
from pinned host memory gives bit-identical logits and tokens to the same
model resident on the GPU, at every prefetch depth; the weights return to
host memory after each module's forward, and the quantizer keeps no
dequantized copy of them (reference weight_offloader.py:48-177,
model_modifier.py:211-268)."""
import copy

import pytest
import torch

from atlasinfer_core.quant import adaptive_quantizer as AQ
from atlasinfer_core.utils import weight_offloader as WO
from integration import atlas_wrappers as AW
from integration import model_modifier as MM

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _llama(seed, layers=3):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    torch.manual_seed(seed)
    m = transformers.LlamaForCausalLM(cfg).half().to(DEV).eval()
    # lm_head quantized too (the embedding stays fp16 and resident)
    MM.apply_atlas_quantization_to_model(m, "llama", {"block_size": -1}, excluded_layers=["embed_tokens"])
    return m


def _streamed_state_on_host(streamer):
    for e in streamer.entries:
        assert not e.installed
        for p in e.params:
            assert p.device.type == "cpu" and p.is_pinned()
        for m, _, _, _ in e.qlinears:
            assert m.quantized_weights.fp8_data.device.type == "cpu"
            assert m.quantized_weights.fp8_data.is_pinned()


@pytest.mark.parametrize("depth", [0, 1, 2])
def test_streamed_llama_forward_matches_resident(depth):
    a = _llama(0)
    b = copy.deepcopy(a)
    streamer = MM.setup_offloading_hooks(b, "llama", torch.device(DEV), prefetch_depth=depth)
    n = len(streamer.entries)
    assert n == 3 + 1 + 1  # blocks, final norm, lm_head
    _streamed_state_on_host(streamer)
    ids = torch.randint(0, 512, (2, 12), device=DEV)
    with torch.no_grad():
        ref = a(ids).logits
        for step in range(2):
            out = b(ids).logits
            assert torch.equal(out, ref)
            _streamed_state_on_host(streamer)
    st = streamer.stats
    if depth == 0:
        assert st["prefetched"] == 0 and st["on_demand"] == 2 * n
    else:
        # only the first module of the first forward is copied on demand
        assert st["on_demand"] == 1 and st["prefetched"] == 2 * n - 1 + depth
    # every module copied once per forward, plus the first `depth` again for a next one
    assert st["bytes"] == 2 * sum(e.nbytes for e in streamer.entries) + sum(
        streamer.entries[k].nbytes for k in range(depth))


def test_streamed_generate_matches_resident():
    a = _llama(1)
    b = copy.deepcopy(a)
    MM.setup_offloading_hooks(b, "llama", torch.device(DEV), prefetch_depth=1)
    ids = torch.randint(0, 512, (1, 8), device=DEV)
    with torch.no_grad():
        ra = a.generate(ids, max_new_tokens=8, do_sample=False, return_dict_in_generate=True, output_logits=True)
        rb = b.generate(ids, max_new_tokens=8, do_sample=False, return_dict_in_generate=True, output_logits=True)
    assert torch.equal(ra.sequences, rb.sequences)
    for la, lb in zip(ra.logits, rb.logits):
        assert torch.equal(la, lb)


def test_device_memory_returns_after_forward():
    a = _llama(2, layers=4)
    streamer = MM.setup_offloading_hooks(a, "llama", torch.device(DEV), prefetch_depth=1)
    ids = torch.randint(0, 512, (1, 8), device=DEV)
    with torch.no_grad():
        a(ids)
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        a(ids)
        torch.cuda.synchronize()
        after = torch.cuda.memory_allocated()
    # between forwards the device holds only the prefetched first block:
    # nothing accumulates from one forward to the next
    assert abs(after - base) < 1 << 20
    assert [i for i, e in enumerate(streamer.entries) if e.dev is not None] == [0]


def test_streamed_opt_with_tied_lm_head():
    transformers = pytest.importorskip("transformers")
    cfg = transformers.OPTConfig(vocab_size=512, hidden_size=256, ffn_dim=512, num_hidden_layers=2,
                                 num_attention_heads=4, max_position_embeddings=64, word_embed_proj_dim=256)
    torch.manual_seed(3)
    a = transformers.OPTForCausalLM(cfg).half().to(DEV).eval()
    MM.apply_atlas_quantization_to_model(a, "opt", {"block_size": -1})  # lm_head excluded: tied, fp16
    b = copy.deepcopy(a)
    streamer = MM.setup_offloading_hooks(b, "opt", torch.device(DEV))
    streamed = {id(e.module) for e in streamer.entries}
    assert id(b.model.decoder.final_layer_norm) in streamed and id(b.lm_head) not in streamed
    assert b.lm_head.weight.device.type == "cuda"
    ids = torch.randint(0, 512, (2, 10), device=DEV)
    with torch.no_grad():
        assert torch.equal(b(ids).logits, a(ids).logits)


def test_reference_flow_model_and_inputs_on_host():
    """The reference's offload run: the whole model in host memory, inputs
    there too; the embedding runs on the CPU, the hooked modules on the
    GPU."""
    transformers = pytest.importorskip("transformers")
    cfg = transformers.OPTConfig(vocab_size=512, hidden_size=256, ffn_dim=512, num_hidden_layers=2,
                                 num_attention_heads=4, max_position_embeddings=64, word_embed_proj_dim=256,
                                 tie_word_embeddings=False)
    torch.manual_seed(4)
    a = transformers.OPTForCausalLM(cfg).half().to(DEV).eval()
    MM.apply_atlas_quantization_to_model(a, "opt", {"block_size": -1}, excluded_layers=["embed_tokens",
                                                                                       "embed_positions"])
    b = copy.deepcopy(a).to("cpu")
    assert b.model.decoder.layers[0].fc1.quantized_weights.fp8_data.device.type == "cpu"
    MM.setup_offloading_hooks(b, "opt", torch.device(DEV))
    ids = torch.randint(0, 512, (1, 10))
    with torch.no_grad():
        ref = a(ids.to(DEV)).logits
        out = b(ids).logits
    assert out.device.type == "cuda"
    rel = ((out.double() - ref.double()).norm() / ref.double().norm()).item()
    assert rel < 1e-3, rel
    with torch.no_grad():
        sa = a.generate(ids.to(DEV), max_new_tokens=6, do_sample=False)
        sb = b.generate(ids, max_new_tokens=6, do_sample=False)
    assert torch.equal(sa.cpu(), sb.cpu())


class _Block(torch.nn.Module):
    def __init__(self, lin, norm):
        super().__init__()
        self.lin = lin
        self.norm = norm

    def forward(self, x):
        return self.lin(self.norm(x))


def _block(seed, N, K):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).half()
    lin = AW.QuantizedLinear(AQ.quantize_tensor(w.to(DEV), block_size=-1),
                             (torch.randn(N, generator=g) * 0.1).half().to(DEV))
    return _Block(lin, torch.nn.LayerNorm(K).half().to(DEV))


def test_hook_without_streamer_moves_weights_there_and_back():
    """The hook alone (no streamer), on a block held in host memory: the
    QuantizedLinear weight and bias go to the GPU for the forward and come
    back after it (the reference's module.to left them behind)."""
    from accelerate.hooks import add_hook_to_module
    blk = _block(5, 256, 512)
    x = torch.randn(4, 512, device=DEV).half()
    with torch.no_grad():
        ref = blk(x)
    blk.to("cpu")
    assert blk.lin.quantized_weights.fp8_data.device.type == "cpu" and blk.lin.bias.device.type == "cpu"
    add_hook_to_module(blk, WO.QuantizedTensorOffloadHook(execution_device=torch.device(DEV), offload=True))
    assert blk.norm.weight.device.type == "cpu"  # init_hook made nothing a meta tensor
    with torch.no_grad():
        y = blk(x)
    assert torch.equal(y, ref)
    assert blk.lin.quantized_weights.fp8_data.device.type == "cpu"
    assert blk.lin.bias.device.type == "cpu" and blk.norm.weight.device.type == "cpu"


def test_dequantized_copies_dropped_after_forward():
    """A weight that does not tile (100 rows) runs dequantize + F.linear,
    which caches the fp16 weight; the streamed forward drops that entry."""
    from accelerate.hooks import add_hook_to_module
    blk = _block(6, 100, 256)
    x = torch.randn(3, 256, device=DEV).half()
    with torch.no_grad():
        ref = blk(x)
    AQ.clear_dequantized_cache()
    streamer = WO.WeightStreamer(DEV, depth=1)
    streamer.register(blk)
    add_hook_to_module(blk, WO.QuantizedTensorOffloadHook(execution_device=streamer.device, offload=True,
                                                          streamer=streamer))
    with torch.no_grad():
        y = blk(x)
    assert torch.equal(y, ref)
    assert len(AQ._dequantized_weights_cache) == 0
