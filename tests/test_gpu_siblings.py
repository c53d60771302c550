"""Sibling groups (q/k/v, gate/up) at decode sizes: one grouped launch for
the first member, the others take its outputs for the same input object;
results within the north-star bounds of the ungrouped layers, and any other
input (another tensor, an in-place change, prefill sizes) computes alone."""
import pytest
import torch

import gpu_ref as R
from atlasinfer_core.quant import adaptive_quantizer as AQ
from integration import atlas_wrappers as AW
from integration import model_modifier as MM

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ql(seed, N, K):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).half()
    m = AW.QuantizedLinear(AQ.quantize_tensor(w.to(DEV), block_size=-1),
                           (torch.randn(N, generator=g) * 0.1).half().to(DEV))
    m._w_ref = R.oracle_reference(m.quantized_weights, w.numpy(), K, "e4m3")
    return m


def _close(y, ref):
    rel = ((y.double() - ref.double()).norm() / ref.double().norm()).item()
    assert rel < 1e-3, rel


def test_group_outputs_match_single_layers():
    q, k, v = _ql(1, 512, 1024), _ql(2, 128, 1024), _ql(3, 128, 1024)
    x = torch.randn(2, 1024, device=DEV).half()
    ref = [AW.qlinear(x, m.quantized_weights, m.bias) for m in (q, k, v)]
    g = AW.SiblingGroup([q, k, v])
    for m in (q, k, v):
        m._group = g
    ys = [q(x), k(x), v(x)]
    for m, y, r in zip((q, k, v), ys, ref):
        _close(y, r)
        R.assert_close(y, R.reference_linear(x, m._w_ref, m.bias), x, m._w_ref)
    assert g.x is None and not g.out  # every kept output consumed
    # a follower on another tensor, or after an in-place change, computes alone
    q(x)
    x2 = x.clone()
    assert torch.equal(k(x2), AW.qlinear(x2, k.quantized_weights, k.bias))
    x.mul_(2)
    assert torch.equal(v(x), AW.qlinear(x, v.quantized_weights, v.bias))
    # prefill sizes take the ordinary path for every member
    xp = torch.randn(100, 1024, device=DEV).half()
    assert torch.equal(q(xp), AW.qlinear(xp, q.quantized_weights, q.bias))


def test_tiny_llama_fused_matches_unfused():
    transformers = pytest.importorskip("transformers")
    cfg = transformers.LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    torch.manual_seed(0)
    a = transformers.LlamaForCausalLM(cfg).half().to(DEV).eval()
    b = transformers.LlamaForCausalLM(cfg).half().to(DEV).eval()
    b.load_state_dict(a.state_dict())
    MM.apply_atlas_quantization_to_model(a, "llama", {"block_size": -1})
    MM.apply_atlas_quantization_to_model(b, "llama", {"block_size": -1}, fuse_siblings=True)
    groups = {id(m._group) for m in b.modules() if type(m).__name__ == "QuantizedLinear" and m._group is not None}
    assert len(groups) == 4  # q/k/v and gate/up in each of 2 layers
    ids = torch.randint(0, 256, (1, 8), device=DEV)
    with torch.no_grad():
        out_a = a.generate(ids, max_new_tokens=6, do_sample=False, return_dict_in_generate=True, output_logits=True)
        out_b = b.generate(ids, max_new_tokens=6, do_sample=False, return_dict_in_generate=True, output_logits=True)
    for la, lb in zip(out_a.logits, out_b.logits):
        rel = ((la.double() - lb.double()).norm() / la.double().norm()).item()
        assert rel < 2e-3, rel


def test_tiny_llama_fused_generate_under_inference_mode():
    """HF pipelines run generate under torch.inference_mode(): inference
    tensors carry no version counter, so the group computes each member
    alone there, with the same results as the unfused model."""
    transformers = pytest.importorskip("transformers")
    cfg = transformers.LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    torch.manual_seed(1)
    a = transformers.LlamaForCausalLM(cfg).half().to(DEV).eval()
    b = transformers.LlamaForCausalLM(cfg).half().to(DEV).eval()
    b.load_state_dict(a.state_dict())
    MM.apply_atlas_quantization_to_model(a, "llama", {"block_size": -1})
    MM.apply_atlas_quantization_to_model(b, "llama", {"block_size": -1}, fuse_siblings=True)
    ids = torch.randint(0, 256, (1, 8), device=DEV)
    with torch.inference_mode():
        out_a = a.generate(ids, max_new_tokens=6, do_sample=False, return_dict_in_generate=True, output_logits=True)
        out_b = b.generate(ids, max_new_tokens=6, do_sample=False, return_dict_in_generate=True, output_logits=True)
    for la, lb in zip(out_a.logits, out_b.logits):
        assert torch.equal(la, lb)
