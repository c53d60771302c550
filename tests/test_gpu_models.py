"""BASELINE configurations 1 and 3 (and a Gemma model) end to end on the GPU:
random-init HF models with every Linear swapped by
apply_atlas_quantization_to_model (integration/model_modifier.py:95-143),
checked against the oracle.

* Each QuantizedLinear's output on the model's own activations (prefill and
  a decode step) is checked by a forward hook against F.linear on the
  oracle-pinned weight (float64, north-star bounds plus the per-element
  bound; tests/gpu_ref.py), on a sample of rows.
* The logits of the prompt match the same model with every QuantizedLinear
  computed as F.linear on those weights (the reference's forward,
  atlas_wrappers.py:56,67) up to the fp16 rounding of 24-32 layers.
* Greedy generate runs to the requested length.

Config 1: OPT-1.3b (24 layers, hidden 2048, 32 heads, FFN 8192, vocab
50272), excluded_layers=[] (lm_head quantized too), 32-token prompt, 128 new
tokens; every weight checked against the oracle in full.  Config 3:
Mistral-7B (32 layers, hidden 4096, 32 / 8 heads, FFN 14336, vocab 32000,
RoPE 1e6), 512-token prompts at batch 1, 8 and 32; every weight (7.0 B
parameters) checked against the oracle in full, the reference weights the
oracle's; greedy
generate runs the config's 256 new tokens at batch 1 and 8 at batch 8 and
32.  Gemma: Gemma-2B's shapes at two layers (the reference's Gemma pattern
set), every Linear swapped and checked against the oracle in full.
Weights: the HF init (N(0, 0.02)) with 0.1 % of each Linear's entries
replaced by +-U(8, 20) * 0.02, as in BASELINE config 0.
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import gpu_ref as R

pytestmark = pytest.mark.gpu
DEV = R.DEV
QCFG = {"block_size": -1, "z_threshold": 3.0, "code_format": "e4m3"}


def plant_outliers(model, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, nn.Linear):
                w = m.weight.view(-1)
                k = int(round(0.001 * w.numel()))
                pos = torch.randperm(w.numel(), generator=g, device=DEV)[:k]
                sign = torch.where(torch.rand(k, generator=g, device=DEV) < 0.5, -1.0, 1.0)
                w[pos] = (sign * (torch.rand(k, generator=g, device=DEV) * 12 + 8) * 0.02).to(w.dtype)


def sample_rows(M, n=16):
    """Rows of x checked by the hooks: first, last and evenly spaced."""
    return sorted(set(np.linspace(0, M - 1, min(n, M)).round().astype(int).tolist()))


class LayerChecks:
    """Forward hooks asserting every QuantizedLinear's output against
    F.linear(x, w_ref, b) in float64 on sampled rows."""

    def __init__(self, model, w_refs):
        self.n = 0
        self.handles = []
        for name, m in model.named_modules():
            if type(m).__name__ == "QuantizedLinear":
                self.handles.append(m.register_forward_hook(self._hook(w_refs[name])))

    def _hook(self, w_ref):
        def hook(mod, inp, out):
            x = inp[0].reshape(-1, w_ref.shape[1])
            y = out.reshape(-1, w_ref.shape[0])
            rows = torch.tensor(sample_rows(x.shape[0]), device=x.device)
            xs = x.index_select(0, rows)
            R.assert_close(y.index_select(0, rows), R.reference_linear(xs, w_ref, mod.bias), xs, w_ref)
            self.n += 1
        return hook

    def remove(self):
        for h in self.handles:
            h.remove()


def reference_logits(model, w_refs, fp32=False, **kw):
    """Logits of the same model with every QuantizedLinear computed as
    F.linear on its reference weight: in fp16 (the reference's forward), or
    in fp32 rounded to fp16 once (another fp32-accumulating implementation,
    whose distance to the first is the noise floor of fp16 rounding through
    the whole model)."""
    from integration import atlas_wrappers as AW
    by_module = {m: w_refs[n] for n, m in model.named_modules() if type(m).__name__ == "QuantizedLinear"}
    saved = AW.QuantizedLinear.forward
    if fp32:
        AW.QuantizedLinear.forward = lambda self, x: F.linear(
            x.float(), by_module[self].float(), None if self.bias is None else self.bias.float()).half()
    else:
        AW.QuantizedLinear.forward = lambda self, x: F.linear(x, by_module[self], self.bias)
    try:
        return model(**kw).logits
    finally:
        AW.QuantizedLinear.forward = saved


def assert_logits_close(logits, model, w_refs, what, **kw):
    """Our logits against the reference's forward on the reference weights,
    within 3x the distance between two equally valid fp32-accumulating
    implementations of that forward (fp16 F.linear and fp32 F.linear rounded
    once), floor 2e-3: the per-linear hooks check each layer against the
    north-star bounds; through 24-32 layers fp16 roundings compound."""
    ref = reference_logits(model, w_refs, **kw)
    ref32 = reference_logits(model, w_refs, fp32=True, **kw)
    rel, floor = rel_l2(logits, ref), rel_l2(ref32, ref)
    print(f"{what}: logits rel-L2 vs F.linear fp16 on the reference weights {rel:.2e} "
          f"(fp32 F.linear vs fp16 F.linear: {floor:.2e})")
    assert rel <= max(3 * floor, 2e-3), (rel, floor)


def rel_l2(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def swap(model, model_type, excluded):
    """Quantize every Linear (weights recorded first) and build each one's
    reference weight: the oracle's, after checking the GPU's quantized
    tensor against it in full."""
    from integration.model_modifier import apply_atlas_quantization_to_model
    kept = {name: m.weight.detach().cpu().numpy() for name, m in model.named_modules()
            if isinstance(m, nn.Linear) and not any(e in name for e in excluded)}
    rep, fail = apply_atlas_quantization_to_model(model, model_type, QCFG, excluded_layers=excluded)
    assert fail == 0
    items = [(name, m.quantized_weights) for name, m in model.named_modules()
             if type(m).__name__ == "QuantizedLinear"]
    assert sorted(n for n, _ in items) == sorted(kept)

    def check(item):
        name, q = item
        return name, R.oracle_reference(q, kept[name], q.original_shape[1], "e4m3")

    # the oracle is C called with the GIL released: eight weights at a time
    # after the first (which loads it)
    w_refs = dict([check(items[0])])
    with ThreadPoolExecutor(max_workers=8) as pool:
        w_refs.update(pool.map(check, items[1:]))
    return rep, w_refs


def test_config1_opt_1_3b_full_swap_generate():
    transformers = pytest.importorskip("transformers")
    cfg = transformers.OPTConfig(num_hidden_layers=24, hidden_size=2048, num_attention_heads=32, ffn_dim=8192,
                                 vocab_size=50272, max_position_embeddings=2048, word_embed_proj_dim=2048)
    torch.manual_seed(0)
    with torch.device(DEV):
        model = transformers.OPTForCausalLM(cfg).half().eval()
    plant_outliers(model, 1)
    rep, w_refs = swap(model, "opt", [])
    assert rep == 24 * 6 + 1  # every Linear, lm_head included
    assert type(model.lm_head).__name__ == "QuantizedLinear"
    g = torch.Generator(device=DEV).manual_seed(3)
    ids = torch.randint(0, cfg.vocab_size, (1, 32), generator=g, device=DEV)
    with torch.no_grad():
        checks = LayerChecks(model, w_refs)
        logits = model(input_ids=ids).logits          # prompt: M = 32
        model(input_ids=ids[:, :1])                   # one token: M = 1
        checks.remove()
        assert checks.n == 2 * rep
        assert_logits_close(logits, model, w_refs, "OPT-1.3b", input_ids=ids)
        out = model.generate(ids, max_new_tokens=128, min_new_tokens=128, do_sample=False, pad_token_id=0)
    assert out.shape == (1, 160)
    assert torch.equal(out[:, :32], ids)


@pytest.fixture(scope="module")
def mistral():
    transformers = pytest.importorskip("transformers")
    cfg = transformers.MistralConfig(num_hidden_layers=32, hidden_size=4096, num_attention_heads=32,
                                     num_key_value_heads=8, head_dim=128, intermediate_size=14336, vocab_size=32000,
                                     rope_theta=1e6, max_position_embeddings=4096)
    torch.manual_seed(0)
    with torch.device(DEV):
        model = transformers.MistralForCausalLM(cfg).half().eval()
    plant_outliers(model, 2)
    rep, w_refs = swap(model, "mistral", ["lm_head", "embed_tokens", "embeddings"])
    assert rep == 32 * 7
    yield cfg, model, rep, w_refs
    del model, w_refs
    torch.cuda.empty_cache()


@pytest.mark.parametrize("B", [1, 8, 32])
def test_config3_mistral_7b(mistral, B):
    cfg, model, rep, w_refs = mistral
    g = torch.Generator(device=DEV).manual_seed(10 + B)
    ids = torch.randint(0, cfg.vocab_size, (B, 512), generator=g, device=DEV)
    with torch.no_grad():
        checks = LayerChecks(model, w_refs)
        out = model(input_ids=ids, use_cache=True)          # prefill: M = 512 B
        nxt = out.logits[:, -1:].argmax(-1)
        model(input_ids=nxt, past_key_values=out.past_key_values, use_cache=True)  # decode step: M = B
        checks.remove()
        assert checks.n == 2 * rep
        assert_logits_close(out.logits, model, w_refs, f"Mistral-7B batch {B}", input_ids=ids)
        del out
        # the config's whole 256 new tokens at batch 1; 8 at the larger batches
        n = 256 if B == 1 else 8
        gen = model.generate(ids, max_new_tokens=n, min_new_tokens=n, do_sample=False, pad_token_id=0)
    assert gen.shape == (B, 512 + n)
    assert torch.equal(gen[:, :512], ids)


def test_gemma_2b_architecture_swap_generate():
    """A Gemma model (the reference's fourth pattern set,
    model_modifier.py:43-48): Gemma-2B's layer shapes (hidden 2048, 8 query
    heads, one key/value head, head_dim 256, GELU-tanh MLP of 16384, vocab
    256000, lm_head tied to the embedding) at two layers.  Every Linear is
    swapped, the tied lm_head [256000, 2048] included; each weight is
    checked against the oracle in full, each layer's output on the prefill
    and on a decode step by the hooks, the prompt's logits against the
    reference's forward, and greedy generate runs.  The swapped model's
    weight bytes (estimate_quantized_model_vram, reference helpers.py:54-82)
    are the QuantizedTensors' components plus the embedding and the norms."""
    transformers = pytest.importorskip("transformers")
    from atlasinfer_core.utils.helpers import estimate_quantized_model_vram
    cfg = transformers.GemmaConfig(num_hidden_layers=2, hidden_size=2048, num_attention_heads=8,
                                   num_key_value_heads=1, head_dim=256, intermediate_size=16384, vocab_size=256000,
                                   hidden_activation="gelu_pytorch_tanh", max_position_embeddings=2048)
    torch.manual_seed(0)
    with torch.device(DEV):
        model = transformers.GemmaForCausalLM(cfg).half().eval()
    assert model.lm_head.weight is model.model.embed_tokens.weight
    plant_outliers(model, 4)
    rep, w_refs = swap(model, "gemma", [])
    assert rep == 2 * 7 + 1
    assert type(model.lm_head).__name__ == "QuantizedLinear"
    qbytes = sum(m.quantized_weights.memory_footprint(include_overhead=False)
                 for m in model.modules() if type(m).__name__ == "QuantizedLinear")
    plain = sum(p.numel() * 2 for n, p in model.named_parameters())  # embedding + norms, fp16
    assert estimate_quantized_model_vram(model) == qbytes + plain
    g = torch.Generator(device=DEV).manual_seed(5)
    ids = torch.randint(0, cfg.vocab_size, (2, 48), generator=g, device=DEV)
    with torch.no_grad():
        checks = LayerChecks(model, w_refs)
        out = model(input_ids=ids, use_cache=True)  # prefill: M = 96
        nxt = out.logits[:, -1:].argmax(-1)
        model(input_ids=nxt, past_key_values=out.past_key_values, use_cache=True)  # decode step: M = 2
        checks.remove()
        assert checks.n == 2 * rep
        assert_logits_close(out.logits, model, w_refs, "Gemma-2B shapes, 2 layers", input_ids=ids)
        gen = model.generate(ids, max_new_tokens=32, min_new_tokens=32, do_sample=False, pad_token_id=0)
    assert gen.shape == (2, 80) and torch.equal(gen[:, :48], ids)
