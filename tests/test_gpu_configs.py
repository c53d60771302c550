"""BASELINE configurations 0, 2 and 4 on the GPU, every result pinned to the
CPU oracle (reference weights from oracle/aq_oracle.c, tests/gpu_ref.py).

* Config 0: one OPT-1.3b decoder layer (q/k/v/out [2048, 2048], fc1
  [8192, 2048], fc2 [2048, 8192], with bias) at the reference's default block
  of 128 in both code formats, and per output channel; M = 1 and 128.
* Config 2: the Llama-3-8B linears at M in {1, 4, 16, 64, 512, 2048}.
* Config 4: Student-t(3) * 0.02 weights with 1 % U(8, 20) * 0.02 outliers at
  the Llama-3-8B MLP shapes and the Gemma-2B lm_head / FFN shapes, M in
  {1, 5, 16, 48, 64, 2048}.  Their 16-row tile rows carry about 1,100
  (K = 4096) to 3,900 (K = 14336) outliers, past the 512 entries the GEMV
  kernels stage in registers / LDS, so these cases run the spill paths
  (entries read from memory in the outlier pass of qlinear_gemv_kernel and
  in the epilogue of qlinear_gemv_x_kernel).
* K >= 65536 with M >= 6: every outlier goes to qlinear_gemv_x_kernel's
  epilogue; a constructed tile row with 3,000+ outliers at every M path.

Reference anchors: quantize_tensor adaptive_quantizer.py:51-148,
dequantize_tensor :156-251, QuantizedLinear.forward atlas_wrappers.py:30-74
(F.linear on the dequantized weight, :56,67).
"""
import numpy as np
import pytest
import torch

import gpu_ref as R
from atlasinfer_amd import _lib
from atlasinfer_core.quant import adaptive_quantizer as AQ
from integration import atlas_wrappers as AW

pytestmark = pytest.mark.gpu
DEV = R.DEV

_cache = {}


def quantized(key, make_w, G, fmt):
    """(q, fp16 numpy weight, oracle reference weight on the GPU) for a
    weight built by make_w(); quantized on the GPU and checked against the
    oracle once per key."""
    if key not in _cache:
        w = make_w()
        q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=G, code_format=fmt)
        Gr = w.shape[1] if G == -1 else G
        _cache[key] = (q, w, R.oracle_reference(q, w, Gr, fmt))
    return _cache[key]


def gpu_weights(N, K, seed, t_dof=None, frac=0.001):
    """BASELINE weights generated on the GPU from a seeded generator (fast at
    Gemma lm_head size), returned as a host fp16 array."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    n = N * K
    if t_dof:
        w = torch.empty(n, device=DEV)
        step = 1 << 26
        for i in range(0, n, step):
            m = min(step, n - i)
            chi = torch.randn(t_dof, m, generator=g, device=DEV).square_().sum(0).div_(t_dof).sqrt_()
            w[i:i + m] = torch.randn(m, generator=g, device=DEV).div_(chi).mul_(0.02)
    else:
        w = torch.randn(n, generator=g, device=DEV) * 0.02
    k = int(round(frac * n))
    pos = torch.randperm(n, generator=g, device=DEV)[:k]
    sign = torch.where(torch.rand(k, generator=g, device=DEV) < 0.5, -1.0, 1.0)
    w[pos] = sign * (torch.rand(k, generator=g, device=DEV) * 12 + 8) * 0.02
    return w.view(N, K).half().cpu().numpy()


def activations(M, K, seed):
    """x ~ N(0, 1) with 4 input channels x30."""
    rng = np.random.default_rng(seed)
    xs = rng.standard_normal((M, K)).astype(np.float32)
    xs[:, rng.permutation(K)[:4]] *= 30
    return torch.from_numpy(xs.astype(np.float16)).to(DEV)


def check_layer(q, w_ref, x, bias=None):
    y = AW.QuantizedLinear(q, bias)(x)
    assert y.dtype == torch.float16 and y.shape == (*x.shape[:-1], w_ref.shape[0])
    R.assert_close(y, R.reference_linear(x, w_ref, bias), x, w_ref)


# ------------------------------------------------------------------ config 0

OPT_LAYER = [("q_proj", 2048, 2048), ("k_proj", 2048, 2048), ("v_proj", 2048, 2048), ("out_proj", 2048, 2048),
             ("fc1", 8192, 2048), ("fc2", 2048, 8192)]


@pytest.mark.parametrize("fmt,G", [("int8", 128), ("e4m3", 128), ("e4m3", -1)])
@pytest.mark.parametrize("name,N,K", OPT_LAYER)
def test_config0_opt_layer(fmt, G, name, N, K):
    """OPT-1.3b layer shapes, N(0, 0.02) + 0.1 % outliers, bias; codes,
    scales and outliers bit-exact against the oracle, outputs at M = 1 and
    128 within the north-star bounds of F.linear on the oracle's weights."""
    seed = sum(map(ord, name))
    q, w, w_ref = quantized(("opt", name, fmt, G), lambda: R.make_weights(np.random.default_rng(seed), (N, K)), G, fmt)
    bias = torch.from_numpy((np.random.default_rng(seed + 1).standard_normal(N) * 0.1).astype(np.float16)).to(DEV)
    for M in (1, 128):
        x = torch.from_numpy(np.random.default_rng(seed + M).standard_normal((M, K)).astype(np.float16)).to(DEV)
        check_layer(q, w_ref, x, bias)


# ------------------------------------------------------------------ config 2

LLAMA = [("q_proj", 4096, 4096), ("k_proj", 1024, 4096), ("gate_proj", 14336, 4096), ("down_proj", 4096, 14336)]


@pytest.mark.parametrize("name,N,K", LLAMA)
def test_config2_llama_linears(name, N, K):
    """Llama-3-8B linears per output channel (E4M3), quantized codes bit-exact
    against the oracle over the whole weight, outputs at every config-2 M
    (and M = 40: three 16-row groups of x in the shared-x GEMV)."""
    seed = 100 + sum(map(ord, name))
    q, w, w_ref = quantized(("llama", name), lambda: gpu_weights(N, K, seed), -1, "e4m3")
    for M in (1, 4, 16, 40, 64, 512, 2048):
        check_layer(q, w_ref, activations(M, K, seed + M))


# ------------------------------------------------------------------ config 4

T3_SHAPES = [("llama_gate", 14336, 4096), ("llama_down", 4096, 14336), ("gemma_lm_head", 256000, 2048),
             ("gemma_gate", 16384, 2048), ("gemma_down", 2048, 16384)]


def tile_row_outliers(q, N):
    rp = q.outlier_row_ptr.cpu().numpy()
    return np.diff(rp[::16])


@pytest.mark.parametrize("name,N,K", T3_SHAPES)
def test_config4_student_t(name, N, K):
    seed = 400 + sum(map(ord, name))
    q, w, w_ref = quantized(("t3", name), lambda: gpu_weights(N, K, seed, t_dof=3, frac=0.01), -1, "e4m3")
    per_tile_row = tile_row_outliers(q, N)
    # heavy tails: tile rows hold more entries than the GEMV kernels stage
    # (every one from K = 4096 on; at K = 2048 about half of them)
    print(f"{name}: outliers per 16-row tile row min {per_tile_row.min()} mean {per_tile_row.mean():.0f} "
          f"max {per_tile_row.max()}")
    if K >= 4096:
        assert per_tile_row.min() > 512, per_tile_row.min()
    else:
        assert (per_tile_row > 512).mean() > 0.2, per_tile_row.mean()
    for M in (1, 5, 16, 48, 64, 2048):
        check_layer(q, w_ref, activations(M, K, seed + M))


def test_config4_quantize_full_8b_layer_shapes_bit_exact():
    """The quantize kernel at config 4's distribution over one Llama-3-8B
    layer's seven weights (q, k, v, o, gate, up, down), each checked in full
    against the oracle (config 4 part 1 quantizes 32 such layers plus the
    embedding and lm_head with the same kernel launches)."""
    for i, (N, K) in enumerate([(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096),
                                (14336, 4096), (4096, 14336)]):
        w = gpu_weights(N, K, 700 + i, t_dof=3, frac=0.01)
        q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=-1, code_format="e4m3")
        R.assert_matches_oracle(q, w, K, "e4m3")


# ------------------------------------------------------- outlier spill paths

def raw_qlinear(q, x, with_lists):
    """aq_qlinear through the C ABI, with or without the block lists (without
    them, 33 <= M <= 64 always takes the shared-x GEMV)."""
    L = _lib.load()
    K = int(q.original_shape[-1])
    N = q.original_shape.numel() // K
    M = x.shape[0]
    codes = AQ.kernel_codes(q, torch.device(DEV))
    tp, te, tmax = AQ.outlier_tiles(q, torch.device(DEV)) if with_lists else (None, None, 0)
    y = torch.empty(M, N, dtype=torch.float16, device=DEV)
    _lib.check(L.aq_qlinear(x.data_ptr(), M, K, N, codes.data_ptr(), q.scale_factors.data_ptr(), q.block_size,
                            _lib.FORMATS[q.code_format], q.outlier_row_ptr.data_ptr(), _lib.ptr(q.outlier_cols),
                            _lib.ptr(q.fp16_outliers), _lib.ptr(tp), _lib.ptr(te), tmax, None, y.data_ptr(), None, 0,
                            _lib.stream_of(torch.device(DEV))), "aq_qlinear")
    return y


@pytest.mark.parametrize("K", [65536, 131072])
def test_gemv_rows_of_64k_and_more(K):
    """K >= 65536: without the block lists the shared-x GEMV adds every
    outlier in its epilogue (the column does not fit its 16-bit LDS entries);
    with them it adds each chunk's outliers by MFMA, its waves' chunk ranges
    reloaded every 64 chunk groups (512 and 1024 chunks of 128 columns, 8
    waves per tile row); the direct GEMV reads x from memory (no LDS copy
    past K = 16384)."""
    N = 64
    G = min(K, 65536)  # aq_max_block_size: rows of 131072 take two blocks
    q, w, w_ref = quantized(("wide", K), lambda: R.make_weights(np.random.default_rng(K), (N, K), frac=0.01, t_dof=3),
                            G, "e4m3")
    for M in (1, 3, 6, 16, 33, 64):
        x = activations(M, K, K + M)
        yref = R.reference_linear(x, w_ref, None)
        R.assert_close(raw_qlinear(q, x, with_lists=False), yref, x, w_ref)
        R.assert_close(raw_qlinear(q, x, with_lists=True), yref, x, w_ref)
    check_layer(q, w_ref, activations(100, K, K + 100))


def crowded_tile_row(rng, N=256, K=4096):
    """Weights whose tile row 2 (rows 32..47) holds 200 planted
    +-U(8, 20) * 0.02 values per row: about 2,500 outliers in one tile row."""
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    for r in range(32, 48):
        cols = rng.permutation(K)[:200]
        w[r, cols] = rng.choice([-1, 1], 200) * rng.uniform(8, 20, 200) * 0.02
    return w.astype(np.float16)


@pytest.mark.parametrize("fmt,G", [("e4m3", -1), ("int8", 128)])
def test_gemv_crowded_tile_row_every_path(fmt, G):
    q, w, w_ref = quantized(("crowd", fmt, G), lambda: crowded_tile_row(np.random.default_rng(11)), G, fmt)
    assert tile_row_outliers(q, 256)[2] > 1500
    for M in (1, 2, 5, 6, 16, 33, 48, 64):
        x = activations(M, 4096, 50 + M)
        yref = R.reference_linear(x, w_ref, None)
        R.assert_close(raw_qlinear(q, x, with_lists=False), yref, x, w_ref)
        R.assert_close(raw_qlinear(q, x, with_lists=True), yref, x, w_ref)


def test_literal_bound_misses_fp16_output_rounding():
    """Why the max-abs check carries one fp16 ulp of the result: on an
    outlier-free layer with |y| up to ~4 max|x| max|w|, torch's own fp16
    F.linear (the reference's forward, atlas_wrappers.py:67) misses the
    literal 2e-3 max|x| max|w| bound against the exact product, and meets
    the bound with the ulp term -- as does the quantized layer."""
    rng = np.random.default_rng(5)
    N, K = 512, 4096
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=-1, code_format="e4m3")
    w_ref = R.oracle_reference(q, w, K, "e4m3")
    x = torch.from_numpy(rng.standard_normal((8, K)).astype(np.float16)).to(DEV)
    exact = R.reference_linear(x, w_ref, None)
    literal = 2e-3 * x.abs().max().double() * w_ref.abs().max().double()
    y_torch = torch.nn.functional.linear(x, w_ref)
    assert (y_torch.double() - exact).abs().max() > literal
    assert ((y_torch.double() - exact).abs() <= R.north_star_abs_bound(exact, x, w_ref)).all()
    check_layer(q, w_ref, x)
