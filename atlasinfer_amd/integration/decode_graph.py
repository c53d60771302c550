"""Greedy decoding with each step captured in one HIP graph.

The reference decodes with HF ``generate`` (examples/run_atlas_inference.py
:244-264), one eager forward per token; on a GPU as fast as this one that
loop is bound by the host (Python and launch overhead), not by the bytes a
token moves.  ``GraphDecoder`` takes a model whose Linears were swapped by
``apply_atlas_quantization_to_model`` (or any HF OPT / Llama / Mistral
model), runs the prompt through the model's own forward, then records one
decode step -- embeddings, every layer (the QuantizedLinear launches, the
attention over a static key/value cache, the norms and activations), the
final norm, the lm_head and the greedy choice -- in a HIP graph and replays
it once per token.

Everything a replay reads that changes from token to token is device
memory updated in place by the graph itself: the current token ``tok``
(written by the argmax at the end of a step), the position ``pos`` (the
index of the key/value slot and of the positional embedding, incremented at
the end of a step), the output slot index, and the key/value cache
(written at ``pos``).  No host value is baked into the graph
except the shapes: batch, cache length, model dimensions.  The host only
guards that a replay never runs past the cache (``max_len``), so no index
leaves its buffer.

With quantized linears the decode GEMVs (``aq_qlinear_decode``) take the
residual adds and the activation: at batch 1 also the norms (the down
projection stages the SwiGLU product as its input), so that a layer is five
launches (six with the attention's span merge); at batch 6 to 64 each norm
is a launch of its own and the gate/up launch writes the SwiGLU product (OPT:
fc1 its ReLU), seven (eight).  Otherwise, on the GPU with an fp16 model, a
layer's step is about nine launches: one
residual add + norm (``aq_decode_norm``) before the attention and one
before the MLP, the q/k/v and gate/up projections as one grouped
QuantizedLinear launch each, the attention (``aq_decode_attention``: query
scaling or rotary embedding, the new key/value written at ``pos``, scores,
softmax and the weighted sum of values over the cache, plus a merge of the
cache spans' partial results), the output projection, the SiLU product
(``aq_silu_mul``) and the down projection.  Elsewhere (CPU, other dtypes,
head sizes other than 64 and 128) the same step runs as torch operations.

Limits: greedy decoding, equal-length prompts without padding (batch rows
share ``pos``), no beam search, no sliding-window attention.
"""
from __future__ import annotations

from typing import Optional

import ctypes

import torch
import torch.nn.functional as F

from .. import _lib


def _kind(model) -> str:
    t = getattr(model.config, "model_type", "")
    if t == "opt":
        return "opt"
    if t in ("llama", "mistral"):
        return "llama"
    raise NotImplementedError(f"GraphDecoder: model type {t!r} (opt, llama, mistral supported)")


class GraphDecoder:
    """Greedy decode of ``model`` for ``batch`` sequences of up to
    ``max_len`` positions (prompt + new tokens), one HIP graph replay per
    token.  ``graph=False`` runs the same step eagerly (no capture), which is
    also how it runs on a CPU."""

    def __init__(self, model, batch: int, max_len: int, graph: bool = True):
        self.model = model
        self.kind = _kind(model)
        cfg = model.config
        self.B, self.L = int(batch), int(max_len)
        p = next(model.parameters())
        self.dev, self.dtype = p.device, p.dtype
        self.use_graph = graph and self.dev.type == "cuda"
        if self.kind == "opt":
            dec = model.model.decoder
            if dec.project_in is not None or dec.project_out is not None or not dec.layers[0].do_layer_norm_before:
                raise NotImplementedError("GraphDecoder: OPT variants with projections or post-norm (350m)")
            self.layers = list(dec.layers)
            self.H = cfg.num_attention_heads
            self.Hkv = self.H
            self.D = cfg.hidden_size // self.H
        else:
            self.layers = list(model.model.layers)
            if getattr(cfg, "sliding_window", None) not in (None, 0) and cfg.sliding_window < self.L:
                raise NotImplementedError("GraphDecoder: sliding-window attention shorter than max_len")
            self.H = cfg.num_attention_heads
            self.Hkv = getattr(cfg, "num_key_value_heads", None) or self.H
            self.D = getattr(cfg, "head_dim", None) or cfg.hidden_size // self.H
        B, L, dev = self.B, self.L, self.dev
        # the state every replay reads and updates in place
        self.tok = torch.zeros(B, dtype=torch.long, device=dev)
        self.pos = torch.zeros(1, dtype=torch.long, device=dev)
        self.slot = torch.zeros(1, dtype=torch.long, device=dev)  # index of the next output token
        self.out = torch.zeros(B, L, dtype=torch.long, device=dev)
        self.logits = None  # the last step's logits (a static buffer once captured)
        self.ar = torch.arange(L, device=dev)
        # keys and values [B, Hkv, L, D]: a position's key is one row
        self.k = [torch.zeros(B, self.Hkv, L, self.D, dtype=self.dtype, device=dev) for _ in self.layers]
        self.v = [torch.zeros(B, self.Hkv, L, self.D, dtype=self.dtype, device=dev) for _ in self.layers]
        if self.kind == "llama":
            rot = model.model.rotary_emb
            pos_ids = torch.arange(L, device=dev)[None]
            with torch.no_grad():
                cos, sin = rot(torch.zeros(1, dtype=self.dtype, device=dev), pos_ids)
            self.cos, self.sin = cos[0].contiguous(), sin[0].contiguous()  # [L, D]
        self.graph = None
        self.captured = False
        self.S, self._n = 0, 0
        # on the GPU: the attention of a step in one HIP kernel
        # (aq_decode_attention), q/k/v and gate/up in one grouped launch each
        self.fused = (self.dev.type == "cuda" and self.dtype == torch.float16 and self.D in (64, 128)
                      and self.H % self.Hkv == 0 and self.H // self.Hkv in (1, 2, 4, 8))
        if self.dev.type == "cuda":
            self._lib = _lib.load()
        if self.fused:
            # the attention kernel's per-span partial results: one workspace
            # for every layer (the layers' calls follow each other on one
            # stream)
            nb = self._lib.aq_decode_attention_workspace(B, self.H, self.Hkv, self.D, L)
            if nb < 0:
                raise ValueError("aq_decode_attention_workspace refused these sizes")
            self.ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=dev)
        # quantized linears at batch 1 or 6..64: SwiGLU / ReLU and residual
        # adds (batch 1: the norms too) folded into the GEMV launches
        # (aq_qlinear_decode)
        self.folded = self._decode_ready()
        self.b1 = self.folded and B == 1
        self.bm = self.folded and B > 1

    # ------------------------------------------------------------ one step

    def _attend_fused(self, li: int, q, k, v, scale: float, q_scale: float, rope: bool):
        """aq_decode_attention: q [B, H, D] scaled by q_scale (rounded to
        fp16) and, with ``rope``, q and the new key k [B, Hkv, D] rotated at
        pos; k, v written at pos; attention over positions 0..pos."""
        B, H, Hkv, D = self.B, self.H, self.Hkv, self.D
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        o = torch.empty(B, H * D, dtype=self.dtype, device=self.dev)
        cs, sn = (self.cos.data_ptr(), self.sin.data_ptr()) if rope else (None, None)
        _lib.check(self._lib.aq_decode_attention(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), self.k[li].data_ptr(), self.v[li].data_ptr(),
            self.pos.data_ptr(), B, H, Hkv, D, self.L, ctypes.c_float(scale), ctypes.c_float(q_scale), cs, sn,
            self.ws.data_ptr(), self.ws.numel(), o.data_ptr(), _lib.stream_of(self.dev)), "aq_decode_attention")
        return o

    def _addnorm(self, x, delta, mod):
        """x += delta in place (fp16 add; none when delta is None), then
        mod(x): one aq_decode_norm launch for HF's Llama/Mistral RMSNorm and
        for LayerNorm with weight and bias, else the torch add and module."""
        rms = type(mod).__name__ in ("LlamaRMSNorm", "MistralRMSNorm")
        if self._norm_folds(mod) and x.shape[-1] % 8 == 0 and x.shape[-1] <= 16384:
            y = torch.empty_like(x)
            eps = mod.variance_epsilon if rms else mod.eps
            _lib.check(self._lib.aq_decode_norm(
                x.data_ptr(), None if delta is None else delta.data_ptr(), mod.weight.data_ptr(),
                None if rms else mod.bias.data_ptr(), ctypes.c_float(eps), x.shape[0], x.shape[-1], 0 if rms else 1,
                y.data_ptr(), _lib.stream_of(self.dev)), "aq_decode_norm")
            return y
        if delta is not None:
            x.add_(delta)
        return mod(x)

    def _silu_mul(self, act, g, u):
        """act(g) * u: one aq_silu_mul launch for SiLU, else torch."""
        if type(act).__name__ in ("SiLU", "SiLUActivation") and g.numel() % 8 == 0:
            out = torch.empty_like(g)
            _lib.check(self._lib.aq_silu_mul(g.data_ptr(), u.data_ptr(), out.data_ptr(), g.numel(),
                                             _lib.stream_of(self.dev)), "aq_silu_mul")
            return out
        return act(g) * u

    # ------------------------- batch 1 and 6..64: GEMVs with prologue and epilogue

    def _norm_folds(self, mod) -> bool:
        """Whether the norm ``mod`` can be the batch-1 GEMV's prologue: HF's
        RMSNorm (Llama / Mistral) or LayerNorm with weight and bias (OPT),
        whose parameters are fp16 [K], contiguous, on the decoder's device
        and 16-byte aligned (the prologue reads them as fp16 pieces of 16
        bytes).  Anything else keeps its own launch or torch module."""
        def param_ok(t):
            return (t is not None and t.dtype == torch.float16 and t.is_contiguous() and t.device == self.dev
                    and t.data_ptr() % 16 == 0)

        if self.kind == "opt":
            return isinstance(mod, torch.nn.LayerNorm) and param_ok(mod.weight) and param_ok(mod.bias)
        return type(mod).__name__ in ("LlamaRMSNorm", "MistralRMSNorm") and param_ok(mod.weight)

    def _decode_ready(self) -> bool:
        """Whether every layer can take the folded form (batch 1 or 6..64):
        all its linears QuantizedLinear weights the fused GEMVs take (at
        batch 1 with K <= 16384), SiLU (Llama / Mistral) or ReLU (OPT)
        between the MLP's linears and, at batch 1, whose norms fold into the
        GEMV: HF's RMSNorm or LayerNorm with bias (OPT)."""
        from .atlas_wrappers import fused_supported
        if not (self.fused and (self.B == 1 or 6 <= self.B <= 64)):
            return False
        b1 = self.B == 1

        def lin_ok(*mods):
            if not all(type(m).__name__ == "QuantizedLinear" for m in mods):
                return False
            qs = [m.quantized_weights for m in mods]
            return (all(fused_supported(q) for q in qs) and len({int(q.original_shape[-1]) for q in qs}) == 1
                    and len({q.code_format for q in qs}) == 1 and (not b1 or int(qs[0].original_shape[-1]) <= 16384))

        def norm_ok(mod):
            return not b1 or self._norm_folds(mod)  # batch 6..64: a launch of its own (_addnorm)

        for layer in self.layers:
            at = layer.self_attn
            if self.kind == "opt":
                ok = (lin_ok(at.q_proj, at.k_proj, at.v_proj) and lin_ok(at.out_proj) and lin_ok(layer.fc1)
                      and lin_ok(layer.fc2) and norm_ok(layer.self_attn_layer_norm) and norm_ok(layer.final_layer_norm)
                      and isinstance(layer.activation_fn, torch.nn.ReLU))
            else:
                ok = (lin_ok(at.q_proj, at.k_proj, at.v_proj) and lin_ok(at.o_proj)
                      and lin_ok(layer.mlp.gate_proj, layer.mlp.up_proj) and lin_ok(layer.mlp.down_proj)
                      and norm_ok(layer.input_layernorm) and norm_ok(layer.post_attention_layernorm)
                      and type(layer.mlp.act_fn).__name__ in ("SiLU", "SiLUActivation"))
            if not ok:
                return False
        return True

    def _qdec(self, mods, x, norm=None, u=None, res=None, relu=None, pair=False):
        """aq_qlinear_decode over ``mods`` (QuantizedLinear sharing x): the
        norm module or the SwiGLU product with u applied to x first, ReLU
        and residual adds on the outputs; ``pair``: mods are (gate, up) and
        the one output is their SwiGLU product."""
        from .atlas_wrappers import PRO_LAYERNORM, PRO_NONE, PRO_RMS, PRO_SWIGLU, qlinear_decode
        qs = [m._weights_on(self.dev) for m in mods]
        for m, q in zip(mods, qs):
            m._ensure_codes(q, self.dev)
        tiles = [m._ensure_tiles(q, self.dev) for m, q in zip(mods, qs)] if self.B > 1 else None
        pro, nw, nb, eps = PRO_NONE, None, None, 0.0
        if norm is not None:
            if isinstance(norm, torch.nn.LayerNorm):
                pro, nw, nb, eps = PRO_LAYERNORM, norm.weight, norm.bias, norm.eps
            else:
                pro, nw, eps = PRO_RMS, norm.weight, norm.variance_epsilon
        elif u is not None:
            pro = PRO_SWIGLU
        return qlinear_decode(x, qs, [m.bias for m in mods], [m._codes for m in mods], pro, u, nw, nb, eps, res,
                              relu, tiles, swiglu_pair=pair)

    def _normed(self, mods, x, norm, relu=None):
        """The linears ``mods`` on norm(x): the norm as the GEMV's prologue
        at batch 1, a launch of its own (aq_decode_norm, no add) at batch
        6..64."""
        if self.B == 1:
            return self._qdec(mods, x, norm=norm, relu=relu)
        return self._qdec(mods, self._addnorm(x, None, norm), relu=relu)

    def _layer_folded(self, li, layer, x):
        """One layer in five launches at batch 1, seven at 6..64 (plus the
        attention's span merge where it splits): [norm,] norm + q/k/v,
        attention, o_proj + residual, [norm,] norm + gate/up (batch 6..64:
        + SwiGLU; OPT: fc1 + ReLU), [SwiGLU +] down + residual (OPT: fc2 +
        residual).  x [B, hidden] is the residual stream; returns the next
        one."""
        B, H, Hkv, D = self.B, self.H, self.Hkv, self.D
        at = layer.self_attn
        if self.kind == "opt":
            q, k, v = self._normed([at.q_proj, at.k_proj, at.v_proj], x, layer.self_attn_layer_norm)
            o = self._attend_fused(li, q.view(B, H, D), k.view(B, Hkv, D), v.view(B, Hkv, D), 1.0, at.scaling,
                                   rope=False)
            x1 = self._qdec([at.out_proj], o, res=[x])[0]
            f = self._normed([layer.fc1], x1, layer.final_layer_norm, relu=[1])[0]
            return self._qdec([layer.fc2], f, res=[x1])[0]
        q, k, v = self._normed([at.q_proj, at.k_proj, at.v_proj], x, layer.input_layernorm)
        o = self._attend_fused(li, q.view(B, H, D), k.view(B, Hkv, D), v.view(B, Hkv, D), at.scaling, 1.0,
                               rope=True)
        x1 = self._qdec([at.o_proj], o, res=[x])[0]
        mlp = layer.mlp
        if self.B > 1:
            h = self._addnorm(x1, None, layer.post_attention_layernorm)
            a = self._qdec([mlp.gate_proj, mlp.up_proj], h, pair=True)[0]
            return self._qdec([mlp.down_proj], a, res=[x1])[0]
        g, u = self._normed([mlp.gate_proj, mlp.up_proj], x1, layer.post_attention_layernorm)
        return self._qdec([mlp.down_proj], g, u=u, res=[x1])[0]

    def _layer_fused(self, li, layer, x, delta):
        """One layer on the GPU path: the residual stream x [B, hidden] is
        updated in place by the norm launches (x += the previous layer's
        output delta, then x += this layer's attention output); returns x
        and the MLP output, which the next norm adds."""
        B, H, Hkv, D = self.B, self.H, self.Hkv, self.D
        at = layer.self_attn
        if self.kind == "opt":
            h = self._addnorm(x, delta, layer.self_attn_layer_norm)
            q, k, v = self._linears([at.q_proj, at.k_proj, at.v_proj], h)
            o = self._attend_fused(li, q.view(B, H, D), k.view(B, Hkv, D), v.view(B, Hkv, D), 1.0, at.scaling,
                                   rope=False)
            h = self._addnorm(x, at.out_proj(o), layer.final_layer_norm)
            return x, layer.fc2(layer.activation_fn(layer.fc1(h)))
        h = self._addnorm(x, delta, layer.input_layernorm)
        q, k, v = self._linears([at.q_proj, at.k_proj, at.v_proj], h)
        o = self._attend_fused(li, q.view(B, H, D), k.view(B, Hkv, D), v.view(B, Hkv, D), at.scaling, 1.0,
                               rope=True)
        h = self._addnorm(x, at.o_proj(o), layer.post_attention_layernorm)
        g, u = self._linears([layer.mlp.gate_proj, layer.mlp.up_proj], h)
        return x, layer.mlp.down_proj(self._silu_mul(layer.mlp.act_fn, g, u))

    def _attend(self, li: int, q, k, v, scale: float = 1.0):
        """Attention of the step's queries q [B, H, D] over positions
        0..pos after writing k, v [B, Hkv, D] at pos (scores rounded to fp16
        as a half-precision product returns them, times ``scale``, softmax
        in f32) -- the torch form of the step."""
        B, H, Hkv, D = self.B, self.H, self.Hkv, self.D
        K, V = self.k[li], self.v[li]
        K.index_copy_(2, self.pos, k.reshape(B, Hkv, 1, D))
        V.index_copy_(2, self.pos, v.reshape(B, Hkv, 1, D))
        qg = q.reshape(B, Hkv, H // Hkv, D)
        s = torch.matmul(qg, K.transpose(2, 3).contiguous()).float()  # [B, Hkv, G, L]
        if scale != 1.0:
            s = s * scale
        s = s.masked_fill(self.ar > self.pos, float("-inf"))
        p = torch.softmax(s, dim=-1).to(self.dtype)
        o = torch.matmul(p, V)  # [B, Hkv, G, D]
        return o.reshape(B, H * D)

    def _linears(self, mods, h):
        """The outputs of several linears on the same input: one grouped
        launch when they are all QuantizedLinear layers the fused kernels
        take (on the GPU), else one call each."""
        from .atlas_wrappers import fused_supported, qlinear_grouped
        if self.dev.type == "cuda" and len(mods) > 1 and all(type(m).__name__ == "QuantizedLinear" for m in mods):
            qs = [m._weights_on(self.dev) for m in mods]
            if (all(fused_supported(q) for q in qs) and len({int(q.original_shape[-1]) for q in qs}) == 1
                    and len({q.code_format for q in qs}) == 1):
                for m, q in zip(mods, qs):
                    m._ensure_codes(q, self.dev)
                return qlinear_grouped(h, qs, [m.bias for m in mods], [m._codes for m in mods])
        return [m(h) for m in mods]

    def _layer_opt(self, li, layer, x):
        at = layer.self_attn
        h = layer.self_attn_layer_norm(x)
        q, k, v = self._linears([at.q_proj, at.k_proj, at.v_proj], h)
        q = q * at.scaling
        B = self.B
        o = self._attend(li, q.view(B, self.H, self.D), k.view(B, self.Hkv, self.D), v.view(B, self.Hkv, self.D))
        x = x + at.out_proj(o)
        h = layer.final_layer_norm(x)
        h = layer.fc2(layer.activation_fn(layer.fc1(h)))
        return x + h

    def _rope(self, t, cos, sin):
        # HF's rotate-half form on [B, heads, D] with cos / sin [D]
        half = t.shape[-1] // 2
        rot = torch.cat((-t[..., half:], t[..., :half]), dim=-1)
        return t * cos + rot * sin

    def _layer_llama(self, li, layer, x):
        at = layer.self_attn
        h = layer.input_layernorm(x)
        B = self.B
        q, k, v = self._linears([at.q_proj, at.k_proj, at.v_proj], h)
        q = q.view(B, self.H, self.D)
        k = k.view(B, self.Hkv, self.D)
        v = v.view(B, self.Hkv, self.D)
        cos = self.cos.index_select(0, self.pos)  # [1, D]
        sin = self.sin.index_select(0, self.pos)
        q = self._rope(q, cos, sin)
        k = self._rope(k, cos, sin)
        o = self._attend(li, q, k, v, at.scaling)
        x = x + at.o_proj(o)
        h = layer.post_attention_layernorm(x)
        g, u = self._linears([layer.mlp.gate_proj, layer.mlp.up_proj], h)
        h = layer.mlp.down_proj(layer.mlp.act_fn(g) * u)
        return x + h

    def _step(self):
        m = self.model
        if self.kind == "opt":
            dec = m.model.decoder
            x = dec.embed_tokens(self.tok)
            x = x + dec.embed_positions.weight.index_select(0, self.pos + 2)
            final, layer_fn = dec.final_layer_norm, self._layer_opt
        else:
            x = m.model.embed_tokens(self.tok)
            final, layer_fn = m.model.norm, self._layer_llama
        if self.folded:
            x = x.contiguous()
            for li, layer in enumerate(self.layers):
                x = self._layer_folded(li, layer, x)
            x = self._addnorm(x, None, final)
        elif self.fused:
            x = x.contiguous()
            delta = None
            for li, layer in enumerate(self.layers):
                x, delta = self._layer_fused(li, layer, x, delta)
            x = self._addnorm(x, delta, final)
        else:
            for li, layer in enumerate(self.layers):
                x = layer_fn(li, layer, x)
            x = final(x)
        logits = m.lm_head(x)  # [B, V]
        nxt = self._argmax(logits)
        self.tok.copy_(nxt)
        self.out.index_copy_(1, self.slot, nxt.view(self.B, 1))
        self.pos.add_(1)
        self.slot.add_(1)
        return logits

    @staticmethod
    def _argmax(logits):
        """Greedy choice (first maximum) in two single-pass reductions over
        short rows: the row split into 64 parts, then the parts' maxima."""
        B, V = logits.shape
        n = 64
        w = (V + n - 1) // n
        x = logits.float()
        if w * n != V:
            x = F.pad(x, (0, w * n - V), value=float("-inf"))
        mx, ix = x.view(B, n, w).max(dim=-1)  # [B, n]
        best, part = mx.max(dim=-1)  # first part holding the maximum
        return part * w + ix.gather(1, part.view(B, 1)).view(B)

    # ------------------------------------------------------------ driving

    def _capture(self):
        """Record one step.  A few eager steps first (allocations, the
        layers' prepared arguments), on scratch positions; the caller's
        prefill then sets the real state."""
        s = torch.cuda.Stream(device=self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s), torch.no_grad():
            for _ in range(2):
                self._step()
        torch.cuda.current_stream(self.dev).wait_stream(s)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph), torch.no_grad():
            self.logits = self._step()
        self.captured = True

    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Run the prompt [B, S] through the model's own forward, fill the
        static cache and set tok / pos / slot; returns the first new token."""
        B, S = input_ids.shape
        if B != self.B or S >= self.L:
            raise ValueError(f"prefill: batch {B} (decoder built for {self.B}), prompt {S} (cache {self.L})")
        if self.use_graph and not self.captured:
            self._capture()
        from transformers import DynamicCache
        cache = DynamicCache()
        out = self.model(input_ids=input_ids.to(self.dev), past_key_values=cache, use_cache=True)
        for li in range(len(self.layers)):
            kl, vl = cache.layers[li].keys, cache.layers[li].values  # [B, Hkv, S, D]
            self.k[li][:, :, :S].copy_(kl)
            self.v[li][:, :, :S].copy_(vl)
        first = self._argmax(out.logits[:, -1])
        self.tok.copy_(first)
        self.out.zero_()
        self.out[:, 0].copy_(first)
        self.pos.fill_(S)
        self.slot.fill_(1)
        self.S, self._n = S, 0
        return first

    @torch.no_grad()
    def step(self) -> torch.Tensor:
        """One decode step (a graph replay when captured): the token chosen
        last goes in at position pos; returns the step's logits [B, V] (the
        static buffer when captured)."""
        # host-side guard: the step writes the cache at pos = S + n and the
        # output at slot 1 + n, both below L
        if self.S + self._n >= self.L:
            raise RuntimeError(f"GraphDecoder: cache of {self.L} positions is full")
        self._n += 1
        if self.use_graph:
            self.graph.replay()
            return self.logits
        self.logits = self._step()
        return self.logits

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int) -> torch.Tensor:
        """Prompt + ``max_new_tokens`` greedy tokens, [B, S + max_new_tokens]."""
        S = input_ids.shape[1]
        if S + max_new_tokens > self.L:
            raise ValueError(f"generate: {S} + {max_new_tokens} positions exceed the cache ({self.L})")
        self.prefill(input_ids)
        for _ in range(max_new_tokens - 1):
            self.step()
        return torch.cat([input_ids.to(self.dev), self.out[:, :max_new_tokens]], dim=1)
