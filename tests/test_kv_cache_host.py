"""Tiered KV cache and attention wrapper on the CPU: the reference's names
and paths, put/get round trips through host memory and the disk tier in
least-recently-used order, and wrapped HF models (Llama, OPT) generating
exactly what the unwrapped models generate, also with a host limit that
sends layers to disk and back between steps (reference
unified_memory_manager.py:111-563, atlas_wrappers.py:84-262,
model_modifier.py:146-208)."""
import copy

import pytest
import torch

import atlasinfer_amd.memory.unified_memory_manager as impl
from atlasinfer_core.memory import unified_memory_manager as UMM
from integration import atlas_wrappers as AW
from integration import model_modifier as MM

CPU = torch.device("cpu")
KiB = 1 / (1024 * 1024)  # in GiB


def _mgr(ram_kib=1024, disk=None, disk_kib=1 << 20):
    return UMM.UnifiedMemoryManager(0, ram_kib * KiB, disk, disk_limit_gb=disk_kib * KiB, gpu_device=CPU)


def test_reference_names_and_paths():
    assert UMM is impl
    for name in ("UnifiedMemoryManager", "KVCacheLayer", "DiskKVStore"):
        assert hasattr(UMM, name)
    assert hasattr(AW, "AtlasAttentionWrapper") and callable(MM.apply_atlas_attention_wrapper)
    m = _mgr()
    for key in ("vram_hits", "ram_hits", "disk_hits", "misses", "evict_vram", "evict_ram", "load_ram",
                "load_disk", "put_vram", "put_ram", "put_disk"):
        assert m.get_stats()[key] == 0
    assert m._get_kv_key(3, "k") == "kv_3_K"


def _kv(seed, S, B=1, H=2, D=8, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, H, S, D, generator=g).to(dtype), torch.randn(B, H, S, D, generator=g).to(dtype)


def test_put_get_round_trip_through_disk_in_lru_order(tmp_path):
    # each layer holds 2 x 2 x 16 x 8 x 2 B = 1 KiB: the host tier takes two
    m = _mgr(ram_kib=2, disk=str(tmp_path / "kv"))
    kvs = {i: _kv(i, 16) for i in range(4)}
    for i in range(3):
        m.put_kv(i, *kvs[i])
    # layer 0 was the least recently used: it went to disk
    assert set(m.ram_cache) == {1, 2} and set(m.disk_entries) == {0}
    k, v = m.get_kv(1)  # touch 1: now 2 is the oldest in host memory
    assert torch.equal(k, kvs[1][0]) and torch.equal(v, kvs[1][1])
    m.put_kv(3, *kvs[3])
    assert set(m.ram_cache) == {1, 3} and set(m.disk_entries) == {0, 2}
    for i in range(4):
        k, v = m.get_kv(i)
        assert torch.equal(k, kvs[i][0]) and torch.equal(v, kvs[i][1]), i
    s = m.get_stats()
    assert s["disk_hits"] >= 2 and s["load_disk"] >= 2 and s["evict_ram"] >= 2 and s["put_disk"] >= 2
    assert m.get_kv(9) == (None, None) and m.get_stats()["misses"] == 1
    files = list((tmp_path / "kv").iterdir())
    m.close()
    assert files and not list((tmp_path / "kv").iterdir())


def test_disk_store_keeps_dtype_and_limit(tmp_path):
    st = UMM.DiskKVStore(str(tmp_path), limit_bytes=64)
    for dt in (torch.float16, torch.bfloat16, torch.float32, torch.int8):
        t = torch.arange(8).to(dt)
        assert st.put("a", t)
        r = st.get("a")
        assert r.dtype == dt and torch.equal(r, t)
    assert not st.put("b", torch.zeros(64, dtype=torch.float32))  # 256 B > 64 B
    assert st.get("b") is None


def test_append_grows_and_equals_concatenation():
    m = _mgr(ram_kib=4096)
    ks, vs = [], []
    for step, q in enumerate([5, 1, 300, 1, 7]):
        k, v = _kv(10 + step, q)
        ks.append(k)
        vs.append(v)
        K, V = m.append_kv(0, k, v)
        assert torch.equal(K, torch.cat(ks, 2)) and torch.equal(V, torch.cat(vs, 2))
    assert m.seq_length(0) == 314 and m.ram_cache[0].k.shape[2] >= 314
    m.truncate(0, 100)
    assert m.seq_length(0) == 100 and torch.equal(m.get_kv(0)[0], torch.cat(ks, 2)[:, :, :100])


def test_crop_follows_hf_dynamic_layer():
    """KVCacheLayer.crop(n) keeps the first n positions and crop(-n) drops n
    from the end, as HF's DynamicLayer.crop; crop(0) empties the layer and a
    length at or past the history changes nothing."""
    m = _mgr(ram_kib=4096)
    k, v = _kv(3, 20)
    layer = UMM.KVCacheLayer(m, 0)
    layer.update(k, v)
    layer.crop(50)
    assert layer.get_seq_length() == 20
    layer.crop(-5)
    assert layer.get_seq_length() == 15 and torch.equal(m.get_kv(0)[0], k[:, :, :15])
    layer.crop(12)
    assert layer.get_seq_length() == 12 and torch.equal(m.get_kv(0)[1], v[:, :, :12])
    layer.crop(0)
    assert layer.get_seq_length() == 0


def test_failed_value_write_leaves_no_key_file(tmp_path):
    """A layer demoted to disk whose keys fit the disk limit but whose
    values do not: the keys' file and its bytes are taken back out, so the
    store holds nothing that no entry owns."""
    # a layer's keys and values are 1 x 2 x 16 x 8 x 2 B = 512 B each: the
    # host tier holds one layer, the disk limit (768 B) its keys only
    m = _mgr(ram_kib=1, disk=str(tmp_path / "kv"), disk_kib=0.75)
    for i in range(2):
        m.put_kv(i, *_kv(i, 16))
    st = m.disk_interface
    assert st.used == 0 and not st.sizes and not list((tmp_path / "kv").iterdir())
    assert 0 not in m.disk_entries
    m.close()


def _tiny(kind, seed):
    transformers = pytest.importorskip("transformers")
    torch.manual_seed(seed)
    if kind == "llama":
        cfg = transformers.LlamaConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=3,
                                       num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=128)
        return transformers.LlamaForCausalLM(cfg).eval()
    cfg = transformers.OPTConfig(vocab_size=256, hidden_size=128, ffn_dim=256, num_hidden_layers=3,
                                 num_attention_heads=4, max_position_embeddings=128, word_embed_proj_dim=128)
    return transformers.OPTForCausalLM(cfg).eval()


@pytest.mark.parametrize("kind", ["llama", "opt"])
@pytest.mark.parametrize("spill", [False, True])
def test_wrapped_model_generates_as_unwrapped(kind, spill, tmp_path):
    a = _tiny(kind, 1)
    b = copy.deepcopy(a)
    # with spill, host memory holds one layer's buffers (256 positions of
    # K and V: 256 KiB for Llama's 2 KV heads, 512 KiB for OPT's 4): the
    # others go to disk and come back at their next step
    one = 256 if kind == "llama" else 512
    m = _mgr(ram_kib=one * 3 // 2 if spill else 4096, disk=str(tmp_path / "kv") if spill else None)
    wrapped, failed = MM.apply_atlas_attention_wrapper(b, kind, m)
    assert (wrapped, failed) == (3, 0)
    assert sorted(a.state_dict()) == sorted(b.state_dict())
    ids = torch.randint(0, 256, (2, 9))
    mask = torch.ones_like(ids)
    with torch.no_grad():
        for _ in range(2):  # a second generate starts a fresh history
            ra = a.generate(ids, attention_mask=mask, max_new_tokens=6, do_sample=False,
                            return_dict_in_generate=True, output_logits=True)
            rb = b.generate(ids, attention_mask=mask, max_new_tokens=6, do_sample=False,
                            return_dict_in_generate=True, output_logits=True)
            assert torch.equal(ra.sequences, rb.sequences)
            for la, lb in zip(ra.logits, rb.logits):
                assert torch.equal(la, lb)
    s = m.get_stats()
    if spill:
        assert s["evict_ram"] > 0 and s["load_disk"] > 0
    else:
        assert s["evict_ram"] == 0 and s["put_ram"] == 2 * 3 * 6
    m.close()
