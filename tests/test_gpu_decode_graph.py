"""GraphDecoder on the GPU with quantized models: every replay of the
captured decode step gives bit-identical logits and tokens to the same step
run eagerly (the eager decoder's work runs between the replays), and the
generated tokens follow HF's own generate on the same quantized model up to
the first near-tie of the top logits (the attention arithmetic differs: f32
scores and softmax here, HF's SDPA there)."""
import copy

import pytest
import torch

from atlasinfer_amd.integration.decode_graph import GraphDecoder
from integration import model_modifier as MM

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _model(kind, seed):
    transformers = pytest.importorskip("transformers")
    torch.manual_seed(seed)
    if kind == "opt":
        cfg = transformers.OPTConfig(vocab_size=512, hidden_size=256, ffn_dim=512, num_hidden_layers=3,
                                     num_attention_heads=4, max_position_embeddings=256, word_embed_proj_dim=256)
        m = transformers.OPTForCausalLM(cfg)
    else:
        cfg = transformers.LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=3,
                                       num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256)
        m = transformers.LlamaForCausalLM(cfg)
    m = m.half().to(DEV).eval()
    MM.apply_atlas_quantization_to_model(m, kind, {"block_size": -1}, excluded_layers=["embed_tokens",
                                                                                      "embed_positions"])
    return m


@pytest.mark.parametrize("kind", ["opt", "llama"])
@pytest.mark.parametrize("batch", [1, 4])
def test_graph_replays_match_eager_steps(kind, batch):
    m = _model(kind, 1)
    ids = torch.randint(0, 512, (batch, 9), device=DEV)
    g = GraphDecoder(m, batch=batch, max_len=40, graph=True)
    e = GraphDecoder(m, batch=batch, max_len=40, graph=False)
    for _ in range(2):  # a second sequence reuses the captured graph
        assert torch.equal(g.prefill(ids), e.prefill(ids))
        for t in range(20):
            lg = g.step().clone()
            le = e.step()
            assert torch.equal(lg, le), t
            assert torch.equal(g.tok, e.tok) and torch.equal(g.pos, e.pos), t
        torch.cuda.synchronize()
        assert torch.equal(g.out, e.out)


@pytest.mark.parametrize("kind", ["opt", "llama"])
def test_graph_generate_follows_hf_generate(kind):
    m = _model(kind, 2)
    ids = torch.randint(0, 512, (2, 12), device=DEV)
    n = 16
    with torch.no_grad():
        ref = m.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=n, do_sample=False,
                         return_dict_in_generate=True, output_logits=True)
    g = GraphDecoder(m, batch=2, max_len=64)
    out = g.generate(ids, n)
    assert out.shape == ref.sequences.shape
    for t in range(n):
        a, b = out[:, 12 + t], ref.sequences[:, 12 + t]
        lg = ref.logits[t].float()
        top2 = lg.topk(2, dim=-1).values
        for row in range(2):
            if a[row] != b[row]:
                # only a near-tie of HF's two best logits may flip the choice
                gap = (top2[row, 0] - top2[row, 1]).item()
                assert gap < 2e-2 * top2[row, 0].abs().item() + 1e-2, (t, row, gap)
                return


@pytest.mark.parametrize("B,H,Hkv,D,L,pos", [(1, 32, 32, 64, 160, 0), (1, 32, 32, 64, 160, 47), (2, 32, 8, 128, 768, 511),
                                             (3, 8, 1, 128, 600, 257), (2, 16, 4, 64, 1000, 999),
                                             (1, 64, 8, 128, 300, 299), (2, 16, 2, 64, 40, 0)])
def test_decode_attention_kernel(B, H, Hkv, D, L, pos):
    """aq_decode_attention against the same attention computed in float64
    from the same fp16 data (scores rounded to fp16 as the kernel's contract
    says); the new key and value land at pos and nothing else in the caches
    changes."""
    import ctypes
    from atlasinfer_amd import _lib
    g = torch.Generator(device=DEV).manual_seed(B * 1000 + pos)
    q = torch.randn(B, H, D, generator=g, device=DEV).half()
    kn = torch.randn(B, Hkv, D, generator=g, device=DEV).half()
    vn = torch.randn(B, Hkv, D, generator=g, device=DEV).half()
    K = torch.randn(B, Hkv, L, D, generator=g, device=DEV).half()
    V = torch.randn(B, Hkv, L, D, generator=g, device=DEV).half()
    K0, V0 = K.clone(), V.clone()
    p = torch.tensor([pos], dtype=torch.long, device=DEV)
    out = torch.empty(B, H, D, dtype=torch.float16, device=DEV)
    scale = D ** -0.5
    _lib.check(_lib.load().aq_decode_attention(q.data_ptr(), kn.data_ptr(), vn.data_ptr(), K.data_ptr(), V.data_ptr(),
                                               p.data_ptr(), B, H, Hkv, D, L, ctypes.c_float(scale), out.data_ptr(),
                                               _lib.stream_of(torch.device(DEV))), "aq_decode_attention")
    torch.cuda.synchronize()
    K0[:, :, pos, :] = kn
    V0[:, :, pos, :] = vn
    assert torch.equal(K, K0) and torch.equal(V, V0)
    G = H // Hkv
    qd = q.double().view(B, Hkv, G, D)
    s = (qd @ K0[:, :, :pos + 1].double().transpose(2, 3)).half().double() * scale  # [B, Hkv, G, pos+1]
    w = torch.softmax(s, dim=-1)
    ref = (w @ V0[:, :, :pos + 1].double()).view(B, H, D)
    err = (out.double() - ref).abs().max().item()
    assert err < 2e-3 * ref.abs().max().item() + 1e-3, err


def test_decode_attention_rejects_group_sizes():
    """Query groups other than 1, 2, 4 and 8 heads per key/value head are
    refused before any launch."""
    from atlasinfer_amd import _lib
    t = torch.zeros(64, dtype=torch.float16, device=DEV)
    p = torch.zeros(1, dtype=torch.long, device=DEV)
    with pytest.raises(_lib.AQError, match="times Hkv"):
        _lib.check(_lib.load().aq_decode_attention(t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(),
                                                   p.data_ptr(), 1, 3, 1, 64, 1, 1.0, t.data_ptr(), None),
                   "aq_decode_attention")
