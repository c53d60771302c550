"""GraphDecoder on the GPU with quantized models: every replay of the
captured decode step gives bit-identical logits and tokens to the same step
run eagerly (the eager decoder's work runs between the replays), and,
teacher-forced with HF's tokens, each step's logits stay within a stated
bound of HF's own generate on the same quantized model at every step (the
attention arithmetic differs: f32 scores and softmax here, HF's SDPA
there)."""
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
@pytest.mark.parametrize("batch", [1, 4, 8])
def test_graph_replays_match_eager_steps(kind, batch):
    m = _model(kind, 1)
    ids = torch.randint(0, 512, (batch, 9), device=DEV)
    g = GraphDecoder(m, batch=batch, max_len=40, graph=True)
    e = GraphDecoder(m, batch=batch, max_len=40, graph=False)
    assert g.b1 == e.b1 == (batch == 1)
    assert g.bm == e.bm == (batch == 8)
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
@pytest.mark.parametrize("batch", [1, 2, 8])
def test_graph_generate_follows_hf_generate(kind, batch):
    """Batch 1 takes the five-launch layers (norms, activation and residual
    adds inside the GEMV launches), batch 2 the nine-launch ones, batch 8
    the seven-launch ones (SwiGLU / ReLU and residual adds inside the GEMV
    launches, the norms apart).

    Teacher-forced against HF's generate on the same quantized model: each
    step is fed HF's token, and its logits must lie within a bound of HF's
    at every one of the n steps (no step is skipped after a near-tie).  The
    bound covers the attention arithmetic, which differs (f32 scores and
    softmax weights here, HF's SDPA in fp16 there): max |d logits| <=
    2e-2 * max |HF logits| per row and step.  Free-running, the decoder's own
    greedy tokens then match HF's wherever HF's two best logits are not
    within that bound of each other."""
    m = _model(kind, 2)
    S, n = 12, 16
    ids = torch.randint(0, 512, (batch, S), device=DEV)
    with torch.no_grad():
        ref = m.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=n, do_sample=False,
                         return_dict_in_generate=True, output_logits=True)
    g = GraphDecoder(m, batch=batch, max_len=64)
    assert g.b1 == (batch == 1) and g.bm == (batch == 8)
    first = g.prefill(ids)
    assert torch.equal(first, ref.sequences[:, S])  # prefill is HF's own forward
    worst = 0.0
    for t in range(1, n):
        g.tok.copy_(ref.sequences[:, S + t - 1])  # HF's token goes in
        lg = g.step().float()
        hf = ref.logits[t].float()
        err = ((lg - hf).abs().amax(-1) / hf.abs().amax(-1)).max().item()
        worst = max(worst, err)
        assert err <= 2e-2, (t, err)
    print(f"{kind} batch {batch}: largest per-step logit difference {worst:.2e} of max |logit|")
    out = g.generate(ids, n)
    assert out.shape == ref.sequences.shape
    for t in range(n):
        hf = ref.logits[t].float()
        top2 = hf.topk(2, dim=-1).values
        same_prefix = torch.all(out[:, S:S + t] == ref.sequences[:, S:S + t], dim=1)
        clear = (top2[:, 0] - top2[:, 1]) > 4e-2 * hf.abs().amax(-1)
        # a row whose earlier tokens all agree and whose best logit is clear
        # of the second must pick HF's token
        must = same_prefix & clear
        assert torch.equal(out[must, S + t], ref.sequences[must, S + t]), t


def _attention_call(lib, q, kn, vn, K, V, pos, ws, scale, q_scale=1.0, cos=None, sin=None):
    import ctypes
    from atlasinfer_amd import _lib
    B, H, D = q.shape
    Hkv, L = K.shape[1], K.shape[2]
    p = torch.tensor([pos], dtype=torch.long, device=DEV)
    out = torch.empty(B, H, D, dtype=torch.float16, device=DEV)
    _lib.check(lib.aq_decode_attention(q.data_ptr(), kn.data_ptr(), vn.data_ptr(), K.data_ptr(), V.data_ptr(),
                                       p.data_ptr(), B, H, Hkv, D, L, ctypes.c_float(scale), ctypes.c_float(q_scale),
                                       None if cos is None else cos.data_ptr(), None if sin is None else sin.data_ptr(),
                                       ws.data_ptr(), ws.numel(), out.data_ptr(), _lib.stream_of(torch.device(DEV))),
               "aq_decode_attention")
    torch.cuda.synchronize()
    return out


def _rope_tables(L, D, theta=10000.0):
    """cos / sin [L, D] in fp16 as HF's rotary embedding builds them."""
    inv = 1.0 / theta ** (torch.arange(0, D, 2, dtype=torch.float32, device=DEV) / D)
    f = torch.outer(torch.arange(L, dtype=torch.float32, device=DEV), inv)
    e = torch.cat((f, f), dim=-1)
    return e.cos().half(), e.sin().half()


@pytest.mark.parametrize("B,H,Hkv,D,L,pos", [(1, 32, 32, 64, 160, 0), (1, 32, 32, 64, 160, 47), (2, 32, 8, 128, 768, 511),
                                             (3, 8, 1, 128, 600, 257), (2, 16, 4, 64, 1000, 999),
                                             (1, 64, 8, 128, 300, 299), (2, 16, 2, 64, 40, 0),
                                             (1, 32, 8, 128, 9000, 8191), (40, 8, 8, 64, 2000, 1500),
                                             (32, 32, 8, 128, 200, 150), (1, 16, 8, 64, 100, 99)])
def test_decode_attention_kernel(B, H, Hkv, D, L, pos):
    """aq_decode_attention against the same attention computed in float64
    from the same fp16 data (scores rounded to fp16 as the kernel's contract
    says); the new key and value land at pos and nothing else in the caches
    changes.  The cases take both ways of splitting the cache: one span per
    head shared by the waves of a workgroup (short caches with little work
    per wave, or 256+ heads x batch rows) and spans merged by a second
    kernel.  A second call on the same workspace at an earlier position
    (fewer spans) checks that nothing of the first call's partial results
    leaks into it."""
    from atlasinfer_amd import _lib
    lib = _lib.load()
    nb = lib.aq_decode_attention_workspace(B, H, Hkv, D, L)
    assert nb > 0
    ws = torch.full((nb,), 0x7f, dtype=torch.uint8, device=DEV)  # no initial contents needed
    g = torch.Generator(device=DEV).manual_seed(B * 1000 + pos)
    K = torch.randn(B, Hkv, L, D, generator=g, device=DEV).half()
    V = torch.randn(B, Hkv, L, D, generator=g, device=DEV).half()
    scale = D ** -0.5
    for p in (pos, pos // 3):
        q = torch.randn(B, H, D, generator=g, device=DEV).half()
        kn = torch.randn(B, Hkv, D, generator=g, device=DEV).half()
        vn = torch.randn(B, Hkv, D, generator=g, device=DEV).half()
        K0, V0 = K.clone(), V.clone()
        out = _attention_call(lib, q, kn, vn, K, V, p, ws, scale)
        K0[:, :, p, :] = kn
        V0[:, :, p, :] = vn
        assert torch.equal(K, K0) and torch.equal(V, V0), p
        _check_attention(q, K0, V0, p, scale, out)


def _check_attention(q, K0, V0, p, scale, out):
    """out against attention over positions 0..p computed in float64 from
    the same fp16 data, the scores rounded to fp16 as the kernel states."""
    B, H, D = q.shape
    Hkv = K0.shape[1]
    qd = q.double().view(B, Hkv, H // Hkv, D)
    s = (qd @ K0[:, :, :p + 1].double().transpose(2, 3)).half().double() * scale  # [B, Hkv, G, p+1]
    w = torch.softmax(s, dim=-1)
    ref = (w @ V0[:, :, :p + 1].double()).view(B, H, D)
    err = (out.double() - ref).abs().max().item()
    assert err < 2e-3 * ref.abs().max().item() + 1e-3, (p, err)


@pytest.mark.parametrize("B,H,Hkv,D,L,pos", [(1, 32, 8, 128, 600, 517), (2, 8, 8, 64, 100, 3)])
def test_decode_attention_rope_and_query_scale(B, H, Hkv, D, L, pos):
    """With rotary tables the kernel rotates q and the new key exactly as
    HF's apply_rotary_pos_emb does in fp16 (the cached key is bit-equal to
    HF's rotated key); a query scale multiplies q in fp16 first, as OPT's
    ``q_proj(x) * scaling``.  The attention itself is then checked as above
    on the rotated / scaled tensors."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    from atlasinfer_amd import _lib
    lib = _lib.load()
    ws = torch.empty(lib.aq_decode_attention_workspace(B, H, Hkv, D, L), dtype=torch.uint8, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(11 + pos)
    K = torch.randn(B, Hkv, L, D, generator=g, device=DEV).half()
    V = torch.randn(B, Hkv, L, D, generator=g, device=DEV).half()
    q = torch.randn(B, H, D, generator=g, device=DEV).half()
    kn = torch.randn(B, Hkv, D, generator=g, device=DEV).half()
    vn = torch.randn(B, Hkv, D, generator=g, device=DEV).half()
    cos, sin = _rope_tables(L, D)
    K0, V0 = K.clone(), V.clone()
    out = _attention_call(lib, q, kn, vn, K, V, pos, ws, D ** -0.5, cos=cos, sin=sin)
    c, s_ = cos[pos].view(1, D), sin[pos].view(1, D)
    qr, kr = apply_rotary_pos_emb(q, kn, c, s_, unsqueeze_dim=0)  # cos / sin broadcast as [1, 1, D]
    assert qr.shape == q.shape and kr.shape == kn.shape
    K0[:, :, pos, :] = kr
    V0[:, :, pos, :] = vn
    assert torch.equal(K, K0) and torch.equal(V, V0)
    _check_attention(qr, K0, V0, pos, D ** -0.5, out)
    # OPT form: q * scaling in fp16, unit score scale, no rotation
    K, V = K0.clone(), V0.clone()
    out = _attention_call(lib, q, kn, vn, K, V, pos, ws, 1.0, q_scale=D ** -0.5)
    K0[:, :, pos, :] = kn
    assert torch.equal(K, K0)
    _check_attention(q * D ** -0.5, K0, V0, pos, 1.0, out)


@pytest.mark.parametrize("mode,rows,n", [(0, 1, 4096), (0, 8, 4096), (0, 3, 2048), (1, 1, 2048), (1, 32, 2048),
                                          (1, 2, 16384), (0, 2, 264)])
def test_decode_norm_matches_hf_modules(mode, rows, n):
    """aq_decode_norm against HF's LlamaRMSNorm (mode 0) and torch's
    LayerNorm (mode 1) modules on the GPU: the residual add is bit-equal to
    torch's fp16 add, the normalised output within one fp16 rounding step
    (the f32 statistics are summed in another order)."""
    import ctypes
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    from atlasinfer_amd import _lib
    lib = _lib.load()
    torch.manual_seed(rows * 7 + n)
    x = (torch.randn(rows, n, device=DEV) * 3).half()
    d = torch.randn(rows, n, device=DEV).half()
    if mode == 0:
        mod = LlamaRMSNorm(n, eps=1e-5).to(DEV).half()
        with torch.no_grad():
            mod.weight.copy_(torch.randn(n, device=DEV).half())
        eps, bias = 1e-5, None
    else:
        mod = torch.nn.LayerNorm(n).to(DEV).half()
        with torch.no_grad():
            mod.weight.copy_(torch.randn(n, device=DEV).half())
            mod.bias.copy_(torch.randn(n, device=DEV).half())
        eps, bias = mod.eps, mod.bias
    for delta in (None, d):
        xk = x.clone()
        y = torch.empty_like(x)
        _lib.check(lib.aq_decode_norm(xk.data_ptr(), None if delta is None else delta.data_ptr(), mod.weight.data_ptr(),
                                      None if bias is None else bias.data_ptr(), ctypes.c_float(eps), rows, n, mode,
                                      y.data_ptr(), _lib.stream_of(torch.device(DEV))), "aq_decode_norm")
        torch.cuda.synchronize()
        xr = x if delta is None else x + delta
        assert torch.equal(xk, xr)
        with torch.no_grad():
            ref = mod(xr)
        err = (y.float() - ref.float()).abs()
        tol = ref.float().abs() * 2.0 ** -10 + 2.0 ** -14
        assert bool((err <= tol).all()), err.max().item()
        assert (y != ref).float().mean().item() < 0.01


def test_silu_mul_matches_torch():
    """aq_silu_mul against torch's fp16 F.silu(g) * u: within one fp16
    rounding step of each op (exp differs in the last f32 bits)."""
    import torch.nn.functional as F
    from atlasinfer_amd import _lib
    lib = _lib.load()
    torch.manual_seed(5)
    g = (torch.randn(3, 14336, device=DEV) * 4).half()
    u = torch.randn(3, 14336, device=DEV).half()
    out = torch.empty_like(g)
    _lib.check(lib.aq_silu_mul(g.data_ptr(), u.data_ptr(), out.data_ptr(), g.numel(), _lib.stream_of(torch.device(DEV))),
               "aq_silu_mul")
    torch.cuda.synchronize()
    ref = F.silu(g) * u
    err = (out.float() - ref.float()).abs()
    assert bool((err <= ref.float().abs() * 2.0 ** -9 + 2.0 ** -20).all()), err.max().item()
    assert (out != ref).float().mean().item() < 0.01


def test_decode_attention_deterministic():
    """The same call twice gives the same bits (the spans' partial results
    are merged in span order)."""
    from atlasinfer_amd import _lib
    lib = _lib.load()
    B, H, Hkv, D, L, pos = 2, 32, 8, 128, 4096, 4000
    ws = torch.zeros(lib.aq_decode_attention_workspace(B, H, Hkv, D, L), dtype=torch.uint8, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(7)
    K = torch.randn(B, Hkv, L, D, generator=g, device=DEV).half()
    V = torch.randn(B, Hkv, L, D, generator=g, device=DEV).half()
    q = torch.randn(B, H, D, generator=g, device=DEV).half()
    kn = torch.randn(B, Hkv, D, generator=g, device=DEV).half()
    vn = torch.randn(B, Hkv, D, generator=g, device=DEV).half()
    a = _attention_call(lib, q, kn, vn, K, V, pos, ws, D ** -0.5)
    for _ in range(3):
        assert torch.equal(_attention_call(lib, q, kn, vn, K, V, pos, ws, D ** -0.5), a)


def test_decode_attention_workspace_checked():
    """A workspace smaller than aq_decode_attention_workspace says is
    refused before any launch."""
    from atlasinfer_amd import _lib
    lib = _lib.load()
    nb = lib.aq_decode_attention_workspace(1, 8, 8, 64, 512)
    t = torch.zeros(max(nb, 4096), dtype=torch.float16, device=DEV)
    p = torch.zeros(1, dtype=torch.long, device=DEV)
    with pytest.raises(_lib.AQError, match="workspace"):
        _lib.check(lib.aq_decode_attention(t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(),
                                           p.data_ptr(), 1, 8, 8, 64, 512, 1.0, 1.0, None, None, t.data_ptr(), nb - 16,
                                           t.data_ptr(), None), "aq_decode_attention")


def test_decode_attention_rejects_group_sizes():
    """Query groups other than 1, 2, 4 and 8 heads per key/value head are
    refused before any launch."""
    from atlasinfer_amd import _lib
    t = torch.zeros(4096, dtype=torch.float16, device=DEV)
    p = torch.zeros(1, dtype=torch.long, device=DEV)
    with pytest.raises(_lib.AQError, match="times Hkv"):
        _lib.check(_lib.load().aq_decode_attention(t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(),
                                                   p.data_ptr(), 1, 3, 1, 64, 1, 1.0, 1.0, None, None, t.data_ptr(),
                                                   8192, t.data_ptr(), None), "aq_decode_attention")
