"""On-disk format of quantized weights (atlasinfer_amd.quant.serialization):
round trips of every QuantizedTensor field, the model-level save/load swap,
and rejection of files that do not match the format.  CPU tests build the
tensors from the oracle (no GPU needed); the GPU test reloads a quantized
model and checks it computes the same logits bit for bit."""
import json

import numpy as np
import pytest
import torch
import torch.nn as nn
from safetensors.torch import save_file

from atlasinfer_amd.quant import serialization as S
from atlasinfer_core.quant import adaptive_quantizer as AQ
from integration import atlas_wrappers as AW


def qt_from_oracle(oracle, w, G, fmt_name):
    """A QuantizedTensor holding the oracle's results for fp16 array w."""
    fmt = oracle.FMT_INT8 if fmt_name == "int8" else oracle.FMT_E4M3
    r = oracle.quantize(w, G, 3.0, fmt)
    N, K = w.shape
    idx = torch.from_numpy(r["outlier_indices"])
    rows = idx // K
    row_ptr = torch.zeros(N + 1, dtype=torch.int32)
    row_ptr[1:] = torch.cumsum(torch.bincount(rows, minlength=N), 0).to(torch.int32)
    if fmt_name == "int8":
        codes = torch.from_numpy(r["fp8_data"])
    else:
        codes = torch.from_numpy(r["codes"]).view(torch.float8_e4m3fn)
    return AQ.QuantizedTensor(codes, torch.from_numpy(r["fp16_outliers"]), idx,
                              torch.from_numpy(r["scale_factors"]), torch.Size(w.shape), G, fmt_name,
                              row_ptr, (idx % K).to(torch.int32))


def weights(seed, shape):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal(shape) * 0.02
    pos = rng.choice(w.size, max(1, w.size // 500), replace=False)
    w.reshape(-1)[pos] = rng.choice([-1.0, 1.0], pos.size) * rng.uniform(8, 20, pos.size) * 0.02
    return w.astype(np.float16)


def same_qt(a, b):
    assert a.original_shape == b.original_shape and a.block_size == b.block_size
    assert (a.code_format, a.code_layout, a.outlier_tile_max) == (b.code_format, b.code_layout, b.outlier_tile_max)
    for f in S._TENSOR_FIELDS:
        x, y = getattr(a, f), getattr(b, f)
        assert (x is None) == (y is None), f
        if x is not None:
            assert x.dtype == y.dtype and x.shape == y.shape, f
            assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), f


@pytest.mark.parametrize("fmt", ["int8", "e4m3"])
@pytest.mark.parametrize("G", [64, 100])
def test_round_trip_fields(tmp_path, oracle, fmt, G):
    qs = {"a": qt_from_oracle(oracle, weights(1, (32, 200)), G, fmt),
          "b": qt_from_oracle(oracle, weights(2, (16, 128)), G, fmt)}
    bias = torch.randn(32).half()
    p = str(tmp_path / "w.safetensors")
    S.save_quantized(qs, p, {"a.bias": bias})
    got, extra = S.load_quantized(p)
    assert set(got) == {"a", "b"} and set(extra) == {"a.bias"}
    for k in qs:
        same_qt(qs[k], got[k])
    assert torch.equal(extra["a.bias"], bias)


def consistent_tiled_qt(seed=0, N=32, K=256, nnz=40):
    """A tiled e4m3 QuantizedTensor with random codes and outliers whose CSR
    and 16 x 64 block lists agree with the flat indices."""
    g = torch.Generator().manual_seed(seed)
    idx = torch.sort(torch.randperm(N * K, generator=g)[:nnz]).values
    vals = torch.randn(nnz, generator=g).half()
    row_ptr = torch.zeros(N + 1, dtype=torch.int32)
    row_ptr[1:] = torch.cumsum(torch.bincount(idx // K, minlength=N), 0).to(torch.int32)
    tp, te = S._block_lists(idx, vals, N, K)
    return AQ.QuantizedTensor(torch.randint(0, 255, (N * K,), dtype=torch.uint8, generator=g).view(torch.float8_e4m3fn),
                              vals, idx, torch.rand(N, generator=g).half(), torch.Size([N, K]), K, "e4m3",
                              row_ptr, (idx % K).to(torch.int32), "tiled", tp,
                              torch.cat([te, torch.zeros(64, dtype=torch.int32)]), int((tp[1:] - tp[:-1]).max()))


def test_round_trip_tiled_and_block_lists(tmp_path):
    """Every optional field (tiled codes, 16 x 64 block lists) survives."""
    q = consistent_tiled_qt()
    p = str(tmp_path / "t.safetensors")
    S.save_quantized({"w": q}, p)
    got, extra = S.load_quantized(p)
    same_qt(q, got["w"])
    assert extra == {}


def test_block_lists_match_expected_tiles_restatement():
    """_block_lists (the loader's check) against the numpy restatement the
    GPU tests use for aq_outlier_tiles."""
    q = consistent_tiled_qt(3, 48, 384, 300)
    N, K = 48, 384
    idx = q.outlier_indices.numpy()
    vals = q.fp16_outliers.numpy().view(np.uint16).astype(np.uint32)
    n, c = idx // K, idx % K
    blk = (n // 16) * (K // 64) + c // 64
    ent = (vals << 16) | (n % 16).astype(np.uint32) << 6 | (c % 64).astype(np.uint32)
    order = np.argsort(blk, kind="stable")
    ptr = np.searchsorted(blk[order], np.arange((N // 16) * (K // 64) + 1))
    assert np.array_equal(q.outlier_tile_ptr.numpy(), ptr)
    assert np.array_equal(q.outlier_tile_ent[:300].numpy().view(np.uint32), ent[order])


CORRUPTIONS = [
    # (field, how to corrupt it, message)
    ("outlier_row_ptr", lambda t: t.flip(0).contiguous(), "CSR pointer"),
    ("outlier_row_ptr", lambda t: t.to(torch.int64), "row pointer dtype"),
    ("outlier_row_ptr", lambda t: torch.cat([t[:1], t[2:], t[-1:]]), "does not match"),
    ("outlier_cols", lambda t: t + 300, "columns do not match"),
    ("outlier_cols", lambda t: t - 1000, "columns do not match"),
    ("outlier_indices", lambda t: t.flip(0).contiguous(), "ascending"),
    ("outlier_indices", lambda t: torch.cat([t[:-1], t[-1:] + (1 << 20)]), "ascending"),
    ("outlier_indices", lambda t: torch.cat([-t[:1] - 1, t[1:]]), "ascending"),
    ("outlier_tile_ptr", lambda t: torch.cat([t[:-1], t[-1:] - 1]), "block lists"),
    ("outlier_tile_ent", lambda t: torch.cat([t[:5] ^ 1, t[5:]]), "block lists"),
    ("outlier_tile_ent", lambda t: t[:-1].contiguous(), "block lists"),
]


@pytest.mark.parametrize("field,corrupt,match", CORRUPTIONS)
def test_corrupted_index_lists_rejected(tmp_path, field, corrupt, match):
    """Index lists that would drive out-of-range or wrong device reads are
    caught on the host before any tensor moves to a device."""
    q = consistent_tiled_qt(1)
    q = q._replace(**{field: corrupt(getattr(q, field))})
    p = str(tmp_path / "c.safetensors")
    S.save_quantized({"w": q}, p)
    with pytest.raises(ValueError, match=match):
        S.load_quantized(p)


def test_understated_tile_max_rejected(tmp_path):
    q = consistent_tiled_qt(2)
    q = q._replace(outlier_tile_max=q.outlier_tile_max - 1)
    p = str(tmp_path / "m.safetensors")
    S.save_quantized({"w": q}, p)
    with pytest.raises(ValueError, match="outlier_tile_max"):
        S.load_quantized(p)


def test_empty_tensor_round_trip(tmp_path):
    q = AQ.quantize_tensor(torch.empty(0, 8, dtype=torch.float16))
    p = str(tmp_path / "e.safetensors")
    S.save_quantized({"e": q}, p)
    same_qt(q, S.load_quantized(p)[0]["e"])


class TwoLayer(nn.Module):
    def __init__(self):
        super().__init__()
        self.block = nn.Sequential(nn.Linear(128, 32), nn.ReLU(), nn.Linear(32, 16, bias=False))
        self.lm_head = nn.Linear(16, 16)


def test_model_save_and_swap(tmp_path, oracle):
    src = TwoLayer()
    q0 = qt_from_oracle(oracle, weights(3, (32, 128)), 128, "e4m3")
    q2 = qt_from_oracle(oracle, weights(4, (16, 32)), 32, "int8")
    b0 = torch.randn(32).half()
    src.block[0] = AW.QuantizedLinear(q0, b0)
    src.block[2] = AW.QuantizedLinear(q2, None)
    p = str(tmp_path / "m.safetensors")
    assert S.save_quantized_model(src, p) == 2
    dst = TwoLayer()
    assert S.load_quantized_model(dst, p) == 2
    assert type(dst.block[0]).__name__ == "QuantizedLinear" and type(dst.lm_head) is nn.Linear
    same_qt(q0, dst.block[0].quantized_weights)
    same_qt(q2, dst.block[2].quantized_weights)
    assert torch.equal(dst.block[0].bias, b0) and dst.block[2].bias is None
    assert dst.lm_head.weight.dtype == torch.float16  # cast as apply_atlas_quantization_to_model does


def test_model_load_rejects_mismatch_before_touching(tmp_path, oracle):
    src = TwoLayer()
    src.block[0] = AW.QuantizedLinear(qt_from_oracle(oracle, weights(5, (32, 128)), 128, "e4m3"), None)
    p = str(tmp_path / "m.safetensors")
    S.save_quantized_model(src, p)
    dst = TwoLayer()  # block.0 has a bias, the file does not
    with pytest.raises(ValueError, match="bias"):
        S.load_quantized_model(dst, p)
    assert type(dst.block[0]) is nn.Linear and dst.block[0].weight.dtype == torch.float32
    other = nn.Module()
    other.block = nn.Sequential(nn.Linear(64, 32))
    with pytest.raises(ValueError, match="shape"):
        S.load_quantized_model(other, p)
    with pytest.raises(ValueError, match="no module"):
        S.load_quantized_model(nn.Module(), p)


def test_foreign_and_inconsistent_files_rejected(tmp_path, oracle):
    p = str(tmp_path / "x.safetensors")
    save_file({"w": torch.zeros(2)}, p)
    with pytest.raises(ValueError, match="not an"):
        S.load_quantized(p)
    q = qt_from_oracle(oracle, weights(6, (16, 128)), 64, "int8")
    good = {f"w/{f}": getattr(q, f).contiguous() for f in S._TENSOR_FIELDS if getattr(q, f) is not None}
    meta = {"format": S.FORMAT_NAME, "version": "1", "entries": json.dumps({"w": S._meta_of(q)})}
    for drop, match in [("w/scale_factors", "lacks"), ("w/fp16_outliers", "lacks")]:
        t = dict(good)
        del t[drop]
        save_file(t, p, metadata=meta)
        with pytest.raises(ValueError, match=match):
            S.load_quantized(p)
    t = dict(good)
    t["w/scale_factors"] = torch.cat([q.scale_factors, q.scale_factors[:1]])
    save_file(t, p, metadata=meta)
    with pytest.raises(ValueError, match="scales"):
        S.load_quantized(p)
    t = dict(good)
    t["v/fp8_data"] = q.fp8_data.clone()
    save_file(t, p, metadata=meta)
    with pytest.raises(ValueError, match="without an entry"):
        S.load_quantized(p)
    save_file(good, p, metadata=dict(meta, version="99"))
    with pytest.raises(ValueError, match="version"):
        S.load_quantized(p)


@pytest.mark.gpu
def test_gpu_reloaded_model_matches(tmp_path):
    transformers = pytest.importorskip("transformers")
    from integration.model_modifier import apply_atlas_quantization_to_model
    dev = "cuda:0"
    cfg = transformers.OPTConfig(vocab_size=256, hidden_size=128, num_hidden_layers=2, ffn_dim=512,
                                 num_attention_heads=4, max_position_embeddings=64, word_embed_proj_dim=128)
    torch.manual_seed(0)
    model = transformers.OPTForCausalLM(cfg).half().to(dev).eval()
    fresh = transformers.OPTForCausalLM(cfg).half().eval()
    fresh.load_state_dict(model.state_dict())
    apply_atlas_quantization_to_model(model, "opt", {"block_size": -1, "z_threshold": 3.0})
    p = str(tmp_path / "opt.safetensors")
    assert S.save_quantized_model(model, p) == 12
    assert S.load_quantized_model(fresh, p, device=dev) == 12
    fresh.to(dev)
    ids = torch.randint(0, 256, (1, 12), device=dev)
    with torch.no_grad():
        a = model(ids).logits
        b = fresh(ids).logits
    assert torch.equal(a, b)
    for (n1, m1), (n2, m2) in zip(model.named_modules(), fresh.named_modules()):
        if type(m1).__name__ == "QuantizedLinear":
            assert n1 == n2
            same_qt(m1.quantized_weights.to("cpu"), m2.quantized_weights.to("cpu"))
