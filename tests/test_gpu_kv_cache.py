"""Tiered KV cache on the GPU: histories appended in place in HBM equal the
concatenation of the steps; put/get round trips through HBM, page-locked
host memory and disk are bit-exact; quantized models with wrapped attention
generate exactly what the unwrapped models generate, with everything in HBM
and with an HBM limit that demotes layers to host memory and disk between
steps (reference unified_memory_manager.py:111-563,
atlas_wrappers.py:84-262)."""
import copy

import pytest
import torch

from atlasinfer_core.memory import unified_memory_manager as UMM
from integration import model_modifier as MM

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
MiB = 1 / 1024


def _kv(seed, S, B=1, H=8, D=128):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(B, H, S, D, generator=g, device=DEV).half(),
            torch.randn(B, H, S, D, generator=g, device=DEV).half())


def test_append_in_hbm_equals_concatenation():
    m = UMM.UnifiedMemoryManager(1.0, 1.0, None, gpu_device=DEV)
    ks, vs = [], []
    for step, q in enumerate([17, 1, 1, 500, 1, 3]):
        k, v = _kv(step, q)
        ks.append(k)
        vs.append(v)
        K, V = m.append_kv(5, k, v)
        assert K.device.type == "cuda"
        assert torch.equal(K, torch.cat(ks, 2)) and torch.equal(V, torch.cat(vs, 2))
    e = m.vram_cache[5]
    assert e.k.shape[2] >= 523 and m.vram_used == 2 * e.k.numel() * 2


def test_put_get_through_host_and_disk(tmp_path):
    # one layer = 2 x 8 x 64 x 128 x 2 B = 256 KiB: HBM takes 2, host memory 2
    m = UMM.UnifiedMemoryManager(0.5 * MiB, 0.5 * MiB, str(tmp_path / "kv"), gpu_device=DEV)
    kvs = {i: _kv(100 + i, 64) for i in range(6)}
    for i in range(6):
        m.put_kv(i, *kvs[i])
    assert set(m.vram_cache) == {4, 5} and set(m.ram_cache) == {2, 3} and set(m.disk_entries) == {0, 1}
    for i in [0, 3, 5, 1, 2, 4]:
        k, v = m.get_kv(i)
        assert k.device.type == "cuda" and torch.equal(k, kvs[i][0]) and torch.equal(v, kvs[i][1]), i
    s = m.get_stats()
    assert s["evict_vram"] > 0 and s["load_ram"] > 0 and s["load_disk"] > 0 and s["disk_hits"] > 0
    m.close()


def _llama(seed):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=3,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256)
    torch.manual_seed(seed)
    m = transformers.LlamaForCausalLM(cfg).half().to(DEV).eval()
    MM.apply_atlas_quantization_to_model(m, "llama", {"block_size": -1})
    return m


@pytest.mark.parametrize("limit", ["hbm", "spill"])
def test_wrapped_quantized_llama_generates_as_unwrapped(limit, tmp_path):
    a = _llama(0)
    b = copy.deepcopy(a)
    if limit == "hbm":
        m = UMM.UnifiedMemoryManager(1.0, 1.0, None, gpu_device=DEV)
    else:
        # a layer's HBM buffers (256 positions, batch 3, 2 KV heads of 64) are
        # 384 KiB: HBM holds one, host memory a few short ones, the rest disk
        m = UMM.UnifiedMemoryManager(0.5 * MiB, 0.3 * MiB, str(tmp_path / "kv"), gpu_device=DEV)
    assert MM.apply_atlas_attention_wrapper(b, "llama", m) == (3, 0)
    ids = torch.randint(0, 512, (3, 11), device=DEV)
    mask = torch.ones_like(ids)
    mask[1, :4] = 0  # a left-padded row
    with torch.no_grad():
        for _ in range(2):
            ra = a.generate(ids, attention_mask=mask, max_new_tokens=8, do_sample=False,
                            return_dict_in_generate=True, output_logits=True)
            rb = b.generate(ids, attention_mask=mask, max_new_tokens=8, do_sample=False,
                            return_dict_in_generate=True, output_logits=True)
            assert torch.equal(ra.sequences, rb.sequences)
            for la, lb in zip(ra.logits, rb.logits):
                assert torch.equal(la, lb)
    s = m.get_stats()
    if limit == "spill":
        assert s["evict_vram"] > 0 and s["load_ram"] + s["load_disk"] > 0
    else:
        assert s["evict_vram"] == 0 and s["vram_cache_items"] == 3
    m.close()
