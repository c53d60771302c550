"""GraphDecoder's decode step on the CPU (eager, no capture): with plain
fp32 OPT, Llama and Mistral models it must generate what HF's own generate
generates, token for token, with the same logits at every step.  This checks
the step's indexing (cache slot, positional embedding and rotary rows at
the device-side position, the causal mask, the output slot) before any
graph is captured on the GPU."""
import pytest
import torch

from atlasinfer_amd.integration.decode_graph import GraphDecoder

transformers = pytest.importorskip("transformers")


def _model(kind):
    torch.manual_seed(0)
    if kind == "opt":
        cfg = transformers.OPTConfig(vocab_size=256, hidden_size=128, ffn_dim=256, num_hidden_layers=2,
                                     num_attention_heads=4, max_position_embeddings=128, word_embed_proj_dim=128)
        return transformers.OPTForCausalLM(cfg).eval()
    cls = transformers.LlamaConfig if kind == "llama" else transformers.MistralConfig
    cfg = cls(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=2, num_attention_heads=4,
              num_key_value_heads=2, max_position_embeddings=128)
    model_cls = transformers.LlamaForCausalLM if kind == "llama" else transformers.MistralForCausalLM
    return model_cls(cfg).eval()


@pytest.mark.parametrize("kind", ["opt", "llama", "mistral"])
def test_eager_step_matches_hf_generate(kind):
    m = _model(kind)
    ids = torch.randint(0, 256, (2, 7))
    with torch.no_grad():
        ref = m.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=10, do_sample=False,
                         return_dict_in_generate=True, output_logits=True)
    gd = GraphDecoder(m, batch=2, max_len=32, graph=False)
    first = gd.prefill(ids)
    assert torch.equal(first, ref.sequences[:, 7])
    for t in range(9):
        lg = gd.step()
        rel = ((lg - ref.logits[t + 1]).abs().max() / ref.logits[t + 1].abs().max()).item()
        assert rel < 1e-5, (t, rel)
    assert torch.equal(gd.generate(ids, 10), ref.sequences)


def test_cache_bound_is_enforced():
    gd = GraphDecoder(_model("opt"), batch=1, max_len=10, graph=False)
    ids = torch.randint(0, 256, (1, 6))
    with pytest.raises(ValueError):
        gd.generate(ids, 5)  # 6 + 5 positions > 10
    gd.prefill(ids)
    for _ in range(4):  # positions 6..9
        gd.step()
    with pytest.raises(RuntimeError):
        gd.step()
    with pytest.raises(ValueError):
        gd.prefill(torch.randint(0, 256, (2, 6)))  # batch differs


def test_unsupported_model_type():
    cfg = transformers.GPT2Config(n_layer=1, n_embd=64, n_head=2, vocab_size=64)
    with pytest.raises(NotImplementedError):
        GraphDecoder(transformers.GPT2LMHeadModel(cfg).eval(), batch=1, max_len=8)


def test_norm_folds_only_fp16_norms():
    """The batch-1 GEMV prologue reads the norm's weight (and LayerNorm's
    bias) as fp16: a norm kept in fp32 or bf16 inside an fp16 model must not
    be folded (nor take aq_decode_norm), whatever its class."""
    for kind in ("opt", "llama"):
        m = _model(kind).half()
        gd = GraphDecoder(m, batch=1, max_len=16, graph=False)
        layer = gd.layers[0]
        norm = layer.self_attn_layer_norm if kind == "opt" else layer.input_layernorm
        assert gd._norm_folds(norm)
        for dt in (torch.float32, torch.bfloat16):
            norm.to(dt)
            assert not gd._norm_folds(norm), (kind, dt)
        norm.half()
        if kind == "opt":
            norm.bias.data = norm.bias.data.float()  # weight fp16, bias not
            assert not gd._norm_folds(norm)
            norm.bias = None
            assert not gd._norm_folds(norm)
