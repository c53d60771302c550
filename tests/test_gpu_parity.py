"""GPU parity: the HIP path against the reference's golden vectors and the
CPU oracle on the same seeded inputs.

Bit-exact: codes, scales, outlier indices/values, dequantized weights,
z-scores.  Tolerance (north star): layer outputs within
max|dy| <= 2e-3 * max|x| * max|w| and ||dy||_2 / ||y||_2 <= 1e-3 of
F.linear(x, W, b) computed in float64, W the oracle's dequantized weight
after the GPU's quantized tensor matched the oracle bit for bit
(tests/gpu_ref.py).
"""
import numpy as np
import pytest
import torch

import gpu_ref as R
from atlasinfer_amd import _lib
from atlasinfer_core.quant import adaptive_quantizer as AQ
from conftest import golden_cases
from gpu_ref import assert_close, bits, make_weights, reference_linear, tile_np
from integration import atlas_wrappers as AW

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
CASES = golden_cases()


def oref(q, w):
    """The oracle's reference weight for GPU tensor ``q`` of weight ``w``
    (bit-exact check of q against the oracle first; tests/gpu_ref.py)."""
    K = int(q.original_shape[-1])
    w16 = np.asarray(w).astype(np.float16).reshape(-1, K)
    return R.oracle_reference(q, w16, q.block_size, q.code_format)


@pytest.mark.parametrize("name,d", CASES, ids=[c[0] for c in CASES])
def test_int8_matches_reference_golden(name, d):
    x = torch.from_numpy(d["x"]).to(DEV)
    q = AQ.quantize_tensor(x, block_size=int(d["block_size"]), z_threshold=float(d["z_threshold"]),
                           code_format="int8")
    assert q.fp8_data.dtype == torch.int8
    assert np.array_equal(bits(q.fp8_data), bits(d["fp8_data"]))
    assert np.array_equal(bits(q.scale_factors), bits(d["scale_factors"]))
    assert np.array_equal(q.outlier_indices.cpu().numpy(), d["outlier_indices"])
    assert np.array_equal(bits(q.fp16_outliers), bits(d["fp16_outliers"]))
    AQ.clear_dequantized_cache()
    deq = AQ.dequantize_tensor(q, torch.device(DEV))
    assert deq.shape == x.shape
    assert np.array_equal(bits(deq), bits(d["deq"]))


def test_cpu_input_returns_on_cpu_and_matches(oracle):
    d = dict(CASES)["opt_like_g128"]
    q = AQ.quantize_tensor(torch.from_numpy(d["x"]), block_size=128, code_format="int8")
    assert q.fp8_data.device.type == "cpu"
    assert np.array_equal(bits(q.fp8_data), bits(d["fp8_data"]))


def test_zscore_matches_reference_golden():
    import os
    from conftest import GOLDEN_DIR
    with np.load(os.path.join(GOLDEN_DIR, "zscore.npz")) as d:
        off = 0
        for n in d["lens"]:
            x = torch.from_numpy(d["x"][off:off + n]).to(DEV)
            z = AQ.calculate_zscore_manual(x)
            assert np.array_equal(bits(z), bits(d["z"][off:off + n])), n
            off += n


SHAPES = [
    # (rows, cols, block, threshold, format, t_dof, outlier fraction)
    (64, 256, 128, 3.0, "e4m3", None, 0.001),
    (48, 512, -1, 3.0, "e4m3", None, 0.001),
    (33, 1000, 100, 3.0, "e4m3", None, 0.01),     # ragged: G does not divide K
    (16, 4096, -1, 3.0, "e4m3", 3, 0.01),
    (8, 14336, -1, 3.0, "int8", None, 0.001),     # per-row block of 14336 (team of 448 x 32), flat codes
    (48, 14336, -1, 3.0, "e4m3", 3, 0.01),        # the same into tiled codes, rows in XCD-contiguous order
    (32, 4096, 128, 3.0, "e4m3", 3, 0.01),        # 32 blocks of 128 (one row) per workgroup, tiled, XCD order
    (32, 8192, -1, 3.0, "e4m3", 3, 0.01),         # two 2-wave teams per workgroup (block-wide votes, paired exchanges)
    (4, 40000, -1, 3.0, "e4m3", None, 0.001),     # block > 16384: 64 elements per thread
    (128, 96, 32, 1.0, "int8", None, 0.05),       # many outliers per block
    # blocks of 33..1024 on teams of 32 elements per thread: full blocks,
    # thread-aligned (G a multiple of 32) and ragged lengths
    (40, 640, 64, 3.0, "e4m3", 3, 0.01),
    (24, 500, 50, 2.0, "int8", None, 0.02),
    (16, 960, 96, 3.0, "e4m3", 3, 0.01),
    (16, 2048, 256, 3.0, "e4m3", 3, 0.01),
    (20, 3000, 300, 2.5, "e4m3", None, 0.01),
    (12, 3072, 1024, 3.0, "e4m3", 3, 0.01),
    (10, 2400, 800, 2.0, "int8", None, 0.01),
    (10, 2100, 700, 3.0, "e4m3", 3, 0.01),
    # count scans over many workgroups: 131 072 blocks (runs of 4 counts per
    # thread) and 2 099 200 blocks (runs of 16), both with outliers in most blocks
    (1024, 4096, 32, 1.0, "e4m3", None, 0.0),
    (8200, 4096, 16, 1.0, "int8", None, 0.0),
    (7, 13, 8, 2.0, "e4m3", None, 0.05),          # G < 16, unaligned rows
    (1, 10, 64, 3.0, "int8", None, 0.0),          # smaller than one block
    (256, 512, 1, 3.0, "int8", None, 0.0),        # G = 1: std is NaN, no outliers
]


@pytest.mark.parametrize("rows,cols,G,thr,fmt,tdof,frac", SHAPES)
def test_quantize_matches_oracle(oracle, rows, cols, G, thr, fmt, tdof, frac):
    rng = np.random.default_rng(rows * 7919 + cols)
    w = make_weights(rng, (rows, cols), frac=frac, t_dof=tdof)
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=G, z_threshold=thr, code_format=fmt)
    Gr = cols if G == -1 else G
    ref = oracle.quantize(w, Gr, thr, oracle.FMT_INT8 if fmt == "int8" else oracle.FMT_E4M3)
    assert q.block_size == Gr
    assert np.array_equal(bits(q.scale_factors), bits(ref["scale_factors"]))
    assert np.array_equal(q.outlier_indices.cpu().numpy(), ref["outlier_indices"])
    assert np.array_equal(bits(q.fp16_outliers), bits(ref["fp16_outliers"]))
    if fmt == "int8":  # the reference's compacted stream
        assert np.array_equal(bits(q.fp8_data), bits(ref["fp8_data"]))
    else:  # dense E4M3 codes, tiled where the shape allows
        assert q.fp8_data.dtype == torch.float8_e4m3fn
        tiled = AQ.tiled_eligible(q.original_shape, Gr)
        assert q.code_layout == ("tiled" if tiled else "flat")
        expect = tile_np(ref["codes"], rows, cols) if tiled else ref["codes"]
        assert np.array_equal(bits(q.fp8_data), expect)
    dense = AQ.dense_codes(q, torch.device(DEV))
    assert np.array_equal(bits(dense), ref["codes"])
    # CSR view of the same outliers
    idx = ref["outlier_indices"]
    inside = idx[idx < rows * cols]
    rp = q.outlier_row_ptr.cpu().numpy()
    assert rp[0] == 0 and rp[-1] == inside.size
    assert np.array_equal(np.diff(rp), np.bincount(inside // cols, minlength=rows))
    assert np.array_equal(q.outlier_cols.cpu().numpy()[: inside.size], (inside % cols).astype(np.int32))
    AQ.clear_dequantized_cache()
    deq = AQ.dequantize_tensor(q, torch.device(DEV))
    assert np.array_equal(bits(deq), bits(oracle.dequantize(ref)))


def test_llama_shape_per_channel_e4m3_full(oracle):
    """A full 4096 x 4096 projection at the product setting (per-channel e4m3)."""
    rng = np.random.default_rng(5)
    w = make_weights(rng, (4096, 4096))
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=-1, code_format="e4m3")
    ref = oracle.quantize(w, 4096, 3.0, oracle.FMT_E4M3)
    assert q.code_layout == "tiled"
    assert np.array_equal(bits(q.fp8_data), tile_np(ref["codes"], 4096, 4096))
    assert np.array_equal(bits(q.scale_factors), bits(ref["scale_factors"]))
    assert np.array_equal(q.outlier_indices.cpu().numpy(), ref["outlier_indices"])


def test_zscore_matches_oracle(oracle):
    rng = np.random.default_rng(1)
    for n in [1, 2, 17, 128, 1000, 4096, 20000, 65536]:
        x = (rng.standard_normal(n) * 0.5).astype(np.float16)
        z = AQ.calculate_zscore_manual(torch.from_numpy(x).to(DEV))
        zr, _ = oracle.zscore(x)
        assert np.array_equal(bits(z), bits(zr)), n


def test_compact_expand_round_trip():
    rng = np.random.default_rng(9)
    w = make_weights(rng, (300, 700), frac=0.02)
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=70, code_format="int8")
    dense = AQ.dense_codes(q, torch.device(DEV))
    qe = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=70, code_format="e4m3")
    assert dense.numel() == qe.fp8_data.numel()
    mask = torch.ones(dense.numel(), dtype=torch.bool, device=DEV)
    mask[q.outlier_indices] = False
    assert torch.equal(dense[mask].view(torch.int8), q.fp8_data)
    assert torch.all(dense[~mask] == 0)


@pytest.mark.parametrize("M", [1, 2, 4, 5, 6, 8, 12, 16, 17, 33, 64, 65, 300])
@pytest.mark.parametrize("fmt,G", [("e4m3", -1), ("int8", 128), ("e4m3", 64), ("e4m3", 128), ("e4m3", 256)])
def test_qlinear_matches_reference_linear(M, fmt, G):
    """Per-channel scales, blocks of 64 (two scales per 128-column chunk) and
    blocks of 128 / 256 (one scale per chunk: the GEMVs' third scale mode)."""
    rng = np.random.default_rng(M + 31 * abs(G))
    N, K = 1024, 2048
    w = make_weights(rng, (N, K))
    xs = rng.standard_normal((M, K)).astype(np.float32)
    xs[:, rng.permutation(K)[:4]] *= 30
    x = torch.from_numpy(xs.astype(np.float16)).to(DEV)
    b = torch.from_numpy((rng.standard_normal(N) * 0.1).astype(np.float16)).to(DEV)
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=G, code_format=fmt)
    w_deq = oref(q, w)
    for bias in (None, b):
        layer = AW.QuantizedLinear(q, bias)
        y = layer(x)
        assert y.shape == (M, N) and y.dtype == torch.float16
        assert_close(y, reference_linear(x, w_deq, bias), x, w_deq)


@pytest.mark.parametrize("N,K", [(1040, 640), (6160, 384), (12304, 384)])
@pytest.mark.parametrize("M", [2, 5, 9, 17, 48, 64])
@pytest.mark.parametrize("fmt,G", [("e4m3", -1), ("int8", 128), ("e4m3", 128)])
def test_gemv_shared_x_ragged_shapes(N, K, M, fmt, G):
    """6 <= M <= 64 (and from M = 2 tall groups with block-wise scales):
    tile-row counts that leave the last workgroup partly empty, chunk counts
    that leave the last chunk group partly past K, and every split width
    (12304 rows take 2 waves per tile row, 6160 take 4, 1040 take 8 up to
    M = 32 and 4 above)."""
    rng = np.random.default_rng(N + K + M + abs(G))
    w = make_weights(rng, (N, K), frac=0.004)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).to(DEV)
    b = torch.from_numpy((rng.standard_normal(N) * 0.1).astype(np.float16)).to(DEV)
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=G, code_format=fmt)
    w_deq = oref(q, w)
    y = AW.QuantizedLinear(q, b)(x)
    assert_close(y, reference_linear(x, w_deq, b), x, w_deq)


@pytest.mark.parametrize("M,N,K", [(2048, 1024, 4096), (512, 4096, 4096), (300, 1024, 2048)])
def test_gemm_split_k_matches_unsplit(M, N, K):
    """Grids too small for the GPU split K and add fp32 partial sums in a
    second kernel (workspace given); without a workspace the same call runs
    unsplit.  Both within the bounds, the split result deterministic."""
    rng = np.random.default_rng(M + N + K)
    w = make_weights(rng, (N, K), frac=0.003)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).to(DEV)
    b = torch.from_numpy((rng.standard_normal(N) * 0.1).astype(np.float16)).to(DEV)
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=-1, code_format="e4m3")
    w_deq = oref(q, w)
    L = _lib.load()
    codes = AQ.kernel_codes(q, torch.device(DEV))
    tp, te, tmax = AQ.outlier_tiles(q, torch.device(DEV))
    ws_bytes = int(L.aq_qlinear_workspace_size(M, N, K))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)

    def run(workspace, nbytes):
        y = torch.empty(M, N, dtype=torch.float16, device=DEV)
        _lib.check(L.aq_qlinear(x.data_ptr(), M, K, N, codes.data_ptr(), q.scale_factors.data_ptr(), K, 1,
                                q.outlier_row_ptr.data_ptr(), q.outlier_cols.data_ptr(), q.fp16_outliers.data_ptr(),
                                tp.data_ptr(), te.data_ptr(), tmax, b.data_ptr(), y.data_ptr(), workspace, nbytes,
                                _lib.stream_of(torch.device(DEV))), "aq_qlinear")
        return y

    ref = reference_linear(x, w_deq, b)
    y_split = run(ws.data_ptr(), ws_bytes)
    y_split2 = run(ws.data_ptr(), ws_bytes)
    y_plain = run(None, 0)
    assert torch.equal(y_split, y_split2)
    assert_close(y_split, ref, x, w_deq)
    assert_close(y_plain, ref, x, w_deq)


@pytest.mark.parametrize("M", [33, 48, 64])
@pytest.mark.parametrize("fmt,G", [("e4m3", -1), ("int8", 128)])
def test_short_grid_gemm_and_gemv_agree_with_reference(M, fmt, G):
    """33 <= M <= 64 on a grid of fewer than 384 tile rows: given the block
    lists (and its workspace) the library runs the GEMM, without them the
    shared-x GEMV; both within the bounds of the reference."""
    N, K = 1040, 1152
    rng = np.random.default_rng(7 * M + abs(G))
    w = make_weights(rng, (N, K), frac=0.004)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).to(DEV)
    b = torch.from_numpy((rng.standard_normal(N) * 0.1).astype(np.float16)).to(DEV)
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=G, code_format=fmt)
    w_deq = oref(q, w)
    L = _lib.load()
    ref = reference_linear(x, w_deq, b)
    y_gemm = AW.qlinear(x, q, b)
    assert_close(y_gemm, ref, x, w_deq)
    codes = AQ.kernel_codes(q, torch.device(DEV))
    y_gemv = torch.empty(M, N, dtype=torch.float16, device=DEV)
    _lib.check(L.aq_qlinear(x.data_ptr(), M, K, N, codes.data_ptr(), q.scale_factors.data_ptr(), q.block_size,
                            _lib.FORMATS[fmt], q.outlier_row_ptr.data_ptr(), q.outlier_cols.data_ptr(),
                            q.fp16_outliers.data_ptr(), None, None, 0, b.data_ptr(), y_gemv.data_ptr(), None, 0,
                            _lib.stream_of(torch.device(DEV))), "aq_qlinear")
    assert_close(y_gemv, ref, x, w_deq)


def test_qlinear_heavy_outliers_and_3d_input():
    rng = np.random.default_rng(77)
    w = make_weights(rng, (512, 1024), frac=0.01, t_dof=3)
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=128, code_format="int8")
    x = torch.from_numpy(rng.standard_normal((2, 3, 1024)).astype(np.float16)).to(DEV)
    b = torch.from_numpy(rng.standard_normal(512).astype(np.float16)).to(DEV)
    w_deq = oref(q, w)
    y = AW.QuantizedLinear(q, b)(x)
    assert y.shape == (2, 3, 512)
    yref = reference_linear(x.reshape(-1, 1024), w_deq, b).reshape(2, 3, 512)
    assert_close(y, yref, x, w_deq)


@pytest.mark.parametrize("fmt,G", [("e4m3", -1), ("int8", 128)])
def test_gemv_m1_crowded_tile_rows(fmt, G):
    """M = 1 with tile rows of more outliers than the GEMV stages (512 a
    tile row: Student-t(3) weights with 5 % heavy outliers give thousands):
    the staged entries summed in the stream, the rest from memory after it."""
    rng = np.random.default_rng(91)
    w = make_weights(rng, (256, 4096), frac=0.05, t_dof=3)
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=G, code_format=fmt)
    rp = q.outlier_row_ptr.cpu().numpy()
    assert (rp[16::16] - rp[:-16:16]).max() > 512  # some tile row overflows the staged entries
    w_deq = oref(q, w)
    b = torch.from_numpy(rng.standard_normal(256).astype(np.float16)).to(DEV)
    for m in (1, 2, 5):
        x = torch.from_numpy(rng.standard_normal((m, 4096)).astype(np.float16)).to(DEV)
        y = AW.QuantizedLinear(q, b)(x)
        assert_close(y, reference_linear(x, w_deq, b), x, w_deq)


def expected_tiles(q, N, K):
    """The 16 x 64 block outlier lists restated with numpy from the flat
    indices: entry (fp16 bits << 16) | r << 6 | k with r = row % 16 and
    k = col % 64, ordered by block (rb * K/64 + col // 64), then row, then column."""
    idx = q.outlier_indices.cpu().numpy()
    vals = bits(q.fp16_outliers).astype(np.uint32)
    n, c = idx // K, idx % K
    blk = (n // 16) * (K // 64) + c // 64
    r, k = (n % 16).astype(np.uint32), (c % 64).astype(np.uint32)
    ent = (vals << 16) | r << 6 | k
    order = np.argsort(blk, kind="stable")  # flat order is already (row, column)
    ptr = np.searchsorted(blk[order], np.arange((N // 16) * (K // 64) + 1))
    return ptr.astype(np.int32), ent[order]


@pytest.mark.parametrize("fmt,G,N,K", [("e4m3", -1, 96, 512), ("int8", 128, 96, 512), ("e4m3", -1, 48, 14336),
                                       ("e4m3", -1, 16, 30720), ("e4m3", 128, 32, 4096), ("e4m3", 32, 16, 30720),
                                       ("e4m3", 4096, 32, 65536), ("int8", 1024, 16, 131072)])
def test_outlier_tiles_match_flat_indices(fmt, G, N, K):
    """aq_outlier_tiles against the block lists rebuilt from the flat
    indices: one workgroup per 16-row tile row up to 480 chunks of 64
    columns (K = 30720), one thread per block beyond (K = 65536, 131072);
    the largest block count, the 64 zeroed padding entries; both on
    heavy-tailed weights (many outliers per block: more than the 1024 a
    workgroup keeps in registers at K = 30720) and on a weight with none.
    E4M3 weights store the lists aq_quantize_finish_tiles builds in the
    same launch as the flat list (per row, several blocks per row with the
    tile row's block offsets in LDS (G = 128) or searched in memory
    (G = 32, K = 30720), and in two launches past 480 chunks): those, and
    that flat list, are checked too."""
    rng = np.random.default_rng(5 + abs(G) + K)
    w = make_weights(rng, (N, K), frac=0.02, t_dof=3)
    for ww in (w, np.zeros_like(w)):
        q = AQ.quantize_tensor(torch.from_numpy(ww).to(DEV), block_size=G, code_format=fmt)
        tp, te, tmax = AQ.build_outlier_tiles(q, torch.device(DEV))
        ptr, ent = expected_tiles(q, N, K)
        nnz = q.outlier_indices.numel()
        assert tmax == (np.diff(ptr).max() if nnz else 0)
        if ww is w:
            assert nnz > 100
        assert np.array_equal(tp.cpu().numpy(), ptr)
        assert te.numel() == nnz + 64
        assert np.array_equal(te[:nnz].cpu().numpy().view(np.uint32), ent)
        assert not te[nnz:].any()
        # the lists quantize_tensor stores (largest count read lazily) are the same
        assert (q.outlier_tile_ptr is not None) == (fmt == "e4m3")
        if q.outlier_tile_ptr is not None:
            assert torch.equal(q.outlier_tile_ptr, tp) and torch.equal(q.outlier_tile_ent, te)
            assert int(q.outlier_tile_max) == tmax
        # the flat list: ascending, the weight's own values, columns and rows
        idx = q.outlier_indices.cpu().numpy()
        assert np.all(np.diff(idx) > 0)
        assert np.array_equal(bits(q.fp16_outliers), ww.reshape(-1).view(np.uint16)[idx])
        assert np.array_equal(q.outlier_cols.cpu().numpy(), idx % K)
        assert np.array_equal(q.outlier_row_ptr.cpu().numpy(), np.searchsorted(idx, np.arange(N + 1) * K))


@pytest.mark.parametrize("M", [17, 65, 200])
def test_gemm_crowded_outlier_blocks(M):
    """Blocks of 16 x 64 holding 0, 1, 9, 17 and 48 outliers: the GEMM reads
    each block's list in batches of 8."""
    rng = np.random.default_rng(900 + M)
    N, K = 256, 1024
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    for (rb, c), per_row in {(0, 0): 3, (1, 5): 1, (3, 15): 2, (7, 2): 1}.items():
        for r in range(16):
            cols = rng.permutation(64)[:per_row] + 64 * c
            w[16 * rb + r, cols] = rng.choice([-1, 1], per_row) * rng.uniform(8, 20, per_row) * 0.02
    w[16 * 5 + 3, 64 * 9 + 7] = 0.4  # a lone outlier
    q = AQ.quantize_tensor(torch.from_numpy(w.astype(np.float16)).to(DEV), block_size=-1, code_format="e4m3")
    tp = q.outlier_tile_ptr.cpu().numpy()
    counts = np.diff(tp).reshape(N // 16, K // 64)
    # the N(0, 0.02) background adds a few outliers of its own
    assert counts[0, 0] >= 48 and counts[3, 15] >= 32 and counts[1, 5] >= 16 and counts[5, 9] >= 1
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).to(DEV)
    w_deq = oref(q, w)
    assert_close(AW.QuantizedLinear(q, None)(x), reference_linear(x, w_deq, None), x, w_deq)


@pytest.mark.parametrize("M,N", [(1000, 4096), (2048, 4096), (2100, 4112)])
def test_gemm_tile_shapes(M, N):
    """Grids of 256 or more 256 x 128 tiles take 256-row tiles (2048 x 4096,
    and 2100 x 4112 with a partial last tile in both directions); smaller
    ones 128-row tiles (1000 x 4096)."""
    rng = np.random.default_rng(M + N)
    K = 1024
    w = make_weights(rng, (N, K))
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=-1, code_format="e4m3")
    xs = rng.standard_normal((M, K)).astype(np.float32)
    xs[:, rng.permutation(K)[:4]] *= 30
    x = torch.from_numpy(xs.astype(np.float16)).to(DEV)
    b = torch.from_numpy((rng.standard_normal(N) * 0.1).astype(np.float16)).to(DEV)
    w_deq = oref(q, w)
    assert_close(AW.QuantizedLinear(q, b)(x), reference_linear(x, w_deq, b), x, w_deq)


@pytest.mark.parametrize("fmt,G,M,N,K", [("e4m3", -1, 2000, 8208, 1024), ("int8", 128, 2048, 8192, 512)])
def test_gemm_wide_tiles(fmt, G, M, N, K):
    """Grids of 256 or more 256 x 256 tiles take the 256 x 256 kernel: a
    partial last M-band and n-tile (2000 x 8208), block-wise int8 scales
    (2048 x 8192), bias, and one 16 x 64 weight block with more than 64
    outliers (read past the first 64 entries)."""
    rng = np.random.default_rng(M + N + K)
    w = make_weights(rng, (N, K)).astype(np.float32)
    for r in range(16):  # 5 per row of block (0, 0): 80 in one block
        cols = rng.permutation(64)[:5]
        w[r, cols] = rng.choice([-1, 1], 5) * rng.uniform(8, 20, 5) * 0.02
    q = AQ.quantize_tensor(torch.from_numpy(w.astype(np.float16)).to(DEV), block_size=G, code_format=fmt)
    assert AQ.outlier_tiles(q, torch.device(DEV))[2] > 64
    xs = rng.standard_normal((M, K)).astype(np.float32)
    xs[:, rng.permutation(K)[:4]] *= 30
    x = torch.from_numpy(xs.astype(np.float16)).to(DEV)
    b = torch.from_numpy((rng.standard_normal(N) * 0.1).astype(np.float16)).to(DEV)
    w_deq = oref(q, w)
    assert_close(AW.QuantizedLinear(q, b)(x), reference_linear(x, w_deq, b), x, w_deq)


@pytest.mark.parametrize("M,N,K", [(256, 8192, 2048), (2048, 16640, 512)])
def test_gemm_wide_tail_in_k_halves(M, N, K):
    """An unsplit 256 x 256 grid whose last round per XCD is at most half
    full runs those tiles as two halves of K, added by a second kernel
    (256 x 8192: every tile; 2048 x 16640: one tile per XCD), given the
    workspace aq_qlinear_workspace_size asks for: against the
    oracle-dequantized reference, and the same call without the workspace
    (whole tiles) within the same bound."""
    assert _lib.load().aq_qlinear_workspace_size(M, N, K) > 0  # the halves are planned
    rng = np.random.default_rng(M * 7 + N)
    w = make_weights(rng, (N, K))
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=-1, code_format="e4m3")
    xs = rng.standard_normal((M, K)).astype(np.float32)
    xs[:, rng.permutation(K)[:4]] *= 30
    x = torch.from_numpy(xs.astype(np.float16)).to(DEV)
    b = torch.from_numpy((rng.standard_normal(N) * 0.1).astype(np.float16)).to(DEV)
    w_deq = oref(q, w)
    ref = reference_linear(x, w_deq, b)
    y = AW.qlinear(x, q, b)
    assert_close(y, ref, x, w_deq)
    tiles = AQ.outlier_tiles(q, torch.device(DEV))
    codes = AQ.kernel_codes(q, torch.device(DEV))
    y0 = torch.empty_like(y)
    _lib.check(_lib.load().aq_qlinear(x.data_ptr(), M, K, N, codes.data_ptr(), q.scale_factors.data_ptr(),
                                      q.block_size, _lib.FORMATS["e4m3"], q.outlier_row_ptr.data_ptr(),
                                      q.outlier_cols.data_ptr(), q.fp16_outliers.data_ptr(), tiles[0].data_ptr(),
                                      tiles[1].data_ptr(), int(tiles[2]), b.data_ptr(), y0.data_ptr(), None, 0,
                                      _lib.stream_of(torch.device(DEV))), "aq_qlinear")
    torch.cuda.synchronize()
    assert_close(y0, ref, x, w_deq)


def test_gemm_dense_outliers_long_rows():
    """Student-t(3) weights with 1% planted outliers (about 2% outliers in
    all) over 14336-wide rows."""
    rng = np.random.default_rng(31)
    N, K, M = 512, 14336, 100
    w = make_weights(rng, (N, K), frac=0.01, t_dof=3)
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=-1, code_format="e4m3")
    assert q.outlier_indices.numel() > 0.015 * N * K
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).to(DEV)
    w_deq = oref(q, w)
    assert_close(AW.QuantizedLinear(q, None)(x), reference_linear(x, w_deq, None), x, w_deq)


def test_qlinear_fallback_for_ragged_blocks():
    """Block 100 does not tile 1000-wide rows: dequantize kernel + F.linear."""
    rng = np.random.default_rng(4)
    w = make_weights(rng, (64, 1000))
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=100, code_format="e4m3")
    x = torch.from_numpy(rng.standard_normal((5, 1000)).astype(np.float16)).to(DEV)
    w_deq = oref(q, w)
    assert_close(AW.QuantizedLinear(q, None)(x), reference_linear(x, w_deq, None), x, w_deq)


def test_qlinear_repeated_calls_are_deterministic():
    rng = np.random.default_rng(12)
    w = make_weights(rng, (1024, 4096))
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=-1)
    x = torch.from_numpy(rng.standard_normal((1, 4096)).astype(np.float16)).to(DEV)
    layer = AW.QuantizedLinear(q, None)
    y0 = layer(x)
    for _ in range(5):
        assert torch.equal(layer(x), y0)


def test_module_to_moves_quantized_weights():
    rng = np.random.default_rng(2)
    w = make_weights(rng, (64, 128))
    q = AQ.quantize_tensor(torch.from_numpy(w), block_size=-1)
    layer = AW.QuantizedLinear(q, torch.zeros(64, dtype=torch.float16))
    layer.to(DEV)
    assert layer.quantized_weights.fp8_data.device.type == "cuda"
    assert layer.bias.device.type == "cuda"


def test_model_swap_tiny_opt():
    transformers = pytest.importorskip("transformers")
    from integration.model_modifier import apply_atlas_quantization_to_model
    cfg = transformers.OPTConfig(vocab_size=256, hidden_size=128, num_hidden_layers=2, ffn_dim=512,
                                 num_attention_heads=4, max_position_embeddings=64, word_embed_proj_dim=128)
    torch.manual_seed(0)
    model = transformers.OPTForCausalLM(cfg).half().to(DEV).eval()
    ids = torch.randint(0, 256, (1, 12), device=DEV)
    before = {n: m.weight.detach().cpu().numpy() for n, m in model.named_modules()
              if isinstance(m, torch.nn.Linear) and n != "lm_head"}
    replaced, failed = apply_atlas_quantization_to_model(model, "opt", {"block_size": -1, "z_threshold": 3.0})
    assert (replaced, failed) == (12, 0)
    qlin = {n: m for n, m in model.named_modules() if type(m).__name__ == "QuantizedLinear"}
    assert sorted(qlin) == sorted(before)
    with torch.no_grad():
        logits = model(ids).logits
        # same model with every QuantizedLinear computed as F.linear on the oracle's weight
        for n, m in qlin.items():
            m._ref_w = oref(m.quantized_weights, before[n])
        saved = AW.QuantizedLinear.forward
        AW.QuantizedLinear.forward = lambda self, x: torch.nn.functional.linear(x, self._ref_w, self.bias)
        try:
            ref = model(ids).logits
        finally:
            AW.QuantizedLinear.forward = saved
    rel = (logits.double() - ref.double()).norm() / ref.double().norm()
    assert rel < 2e-3, rel.item()
    out = model.generate(ids, max_new_tokens=4, do_sample=False)
    assert out.shape == (1, 16)


def test_signed_zeros_survive(oracle):
    """-0 weights and tiny negative weights quantize to the E4M3 code 0x80
    (negative zero) and dequantize to -0; z-scores of -0 inputs stay -0."""
    w = np.zeros((4, 64), np.float16)
    w[:, 0] = 0.5
    w[:, 1] = -0.5
    w[0, 2:10] = np.float16(-0.0)
    w[1, 2:10] = np.float16(-1e-7)   # |x| / s below half the smallest E4M3 step
    w[2, 2:10] = np.float16(1e-7)
    for fmt, ofmt in [("e4m3", oracle.FMT_E4M3), ("int8", oracle.FMT_INT8)]:
        q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=64, code_format=fmt)
        ref = oracle.quantize(w, 64, 3.0, ofmt)
        assert np.array_equal(bits(AQ.dense_codes(q, torch.device(DEV))), ref["codes"])
        AQ.clear_dequantized_cache()
        deq = AQ.dequantize_tensor(q, torch.device(DEV))
        assert np.array_equal(bits(deq), bits(oracle.dequantize(ref)))
    x = np.array([-0.0, 0.0, 1.0, -1.0] * 8, np.float16)
    z = AQ.calculate_zscore_manual(torch.from_numpy(x).to(DEV))
    zr, _ = oracle.zscore(x)
    assert np.array_equal(bits(z), bits(zr))


@pytest.mark.parametrize("G,rows,K", [(128, 64, 4096), (4096, 64, 4096), (14336, 32, 14336)])
def test_quantize_block_means_near_fp16_ties(oracle, G, rows, K):
    """Blocks whose exact mean sits within a few 2^-24 / G of the midpoint of
    two fp16 neighbours h1 < h2 ~ 2^-13 (mean = h1 + 2^-24 + d 2^-24 / G,
    d in -3..3), the rest of each block cancelling pairs +-B with B up to
    6e4, so fp32 partial sums of the block lose the small terms: every
    block's mean16, and so its codes and outliers, must be the oracle's.
    Rows of 14336 run on a team of 7 waves whose sums pad an eighth with +0."""
    rng = np.random.default_rng(G)
    nb = rows * K // G
    w = np.zeros((nb, G), np.float16)
    # h1 * G must be an fp16 value: any h1 for a power-of-two G; at
    # G = 14336 = 7 * 2^11 (products near 1.75, ulp 2^-10) h1's offset a
    # multiple of 4 * 2^-23
    steps = rng.integers(0, 1023, nb) if G & (G - 1) == 0 else 4 * rng.integers(0, 36, nb)
    h1 = np.float16(2.0 ** -13) + np.float16(2.0 ** -23) * steps.astype(np.float16)
    assert np.all(np.float16(h1 * np.float16(G)).astype(np.float64) == h1.astype(np.float64) * G)
    d = rng.integers(-3, 4, nb)
    npair = (G - 4) // 2
    big = (rng.uniform(1.0, 6e4, (nb, npair)) * rng.choice([1e-4, 1.0], (nb, 1))).astype(np.float16)
    vals = np.concatenate([h1[:, None] * np.float16(G), np.full((nb, 1), np.float16(2.0 ** -24 * G)),
                           (d * 2.0 ** -24).astype(np.float16)[:, None], np.zeros((nb, 1), np.float16),
                           big, -big], axis=1)
    for i in range(nb):
        w[i] = vals[i, rng.permutation(G)]
    w = w.reshape(rows, K)
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=G, z_threshold=3.0, code_format="e4m3")
    ref = oracle.quantize(w, G, 3.0, oracle.FMT_E4M3)
    assert np.array_equal(bits(q.scale_factors), bits(ref["scale_factors"]))
    assert np.array_equal(q.outlier_indices.cpu().numpy(), ref["outlier_indices"])
    assert np.array_equal(bits(q.fp16_outliers), bits(ref["fp16_outliers"]))
    assert np.array_equal(bits(AQ.dense_codes(q, torch.device(DEV))), ref["codes"])
    z = AQ.calculate_zscore_manual(torch.from_numpy(w[0, :G].copy()).to(DEV))
    zr, _ = oracle.zscore(w[0, :G])
    assert np.array_equal(bits(z), bits(zr))


def test_e4m3_codes_every_fp16_value(oracle):
    """Every fp16 value in [-448, 448] quantized with scale 1 (each row holds
    448, so amax / 448 = 1) and no outliers (threshold 60000): each code is
    the E4M3 encoding of the value itself, checked against the oracle's
    round-to-nearest-even encoder for all 48 642 values."""
    pos = np.arange(0, 0x5F01, dtype=np.uint16)  # +0 .. 448
    vals = np.concatenate([pos, pos | 0x8000]).view(np.float16)
    K = 1024
    rows = -(-vals.size // (K - 1))
    rows += (-rows) % 16
    w = np.zeros((rows, K), np.float16)
    flat = w[:, 1:].reshape(-1)
    flat[:vals.size] = vals
    w[:, 1:] = flat.reshape(rows, K - 1)
    w[:, 0] = 448.0
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=-1, z_threshold=60000.0, code_format="e4m3")
    assert q.outlier_indices.numel() == 0 and q.code_layout == "tiled"
    assert np.all(bits(q.scale_factors) == 0x3C00)  # 1.0
    ref = oracle.quantize(w, K, 60000.0, oracle.FMT_E4M3)
    assert np.array_equal(bits(AQ.dense_codes(q, torch.device(DEV))), ref["codes"])


def test_e4m3_quotients_above_448(oracle):
    """Block maxima whose quotient x / s exceeds 448: with s = fp16(amax /
    448) rounded down (most of all where s is an fp16 subnormal) amax / s
    reaches 461.  Every positive fp16 amax with fp16(amax / s) > 448 (an
    exhaustive search, 4379 values) gets a row holding +amax and -amax;
    their codes must be the E4M3 encodings of the quotient clamped to
    +-448 (0x7E, 0xFE), as in the oracle."""
    vals = np.arange(0x0400, 0x7C00, dtype=np.uint16).view(np.float16)
    a = vals.astype(np.float32)
    s = np.maximum((a / np.float32(448)).astype(np.float16), np.float16(1e-6))
    hit = vals[(a / s.astype(np.float32)).astype(np.float16) > 448]
    assert hit.size > 4000
    K = 128
    rows = hit.size + (-hit.size) % 16
    w = np.zeros((rows, K), np.float16)
    w[:hit.size, 0] = hit
    w[:hit.size, 1] = -hit
    w[hit.size:, 0] = 1.0
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=-1, z_threshold=60000.0, code_format="e4m3")
    assert q.outlier_indices.numel() == 0
    ref = oracle.quantize(w, K, 60000.0, oracle.FMT_E4M3)
    got = bits(AQ.dense_codes(q, torch.device(DEV))).reshape(rows, K)
    assert np.array_equal(got, ref["codes"].reshape(rows, K))
    assert np.all(got[:hit.size, 0] == 0x7E) and np.all(got[:hit.size, 1] == 0xFE)


def test_tile_untile_round_trip():
    from atlasinfer_amd import _lib
    L = _lib.load()
    rng = np.random.default_rng(21)
    N, K = 48, 384
    flat = torch.from_numpy(rng.integers(0, 256, N * K).astype(np.uint8)).to(DEV)
    tiled = torch.empty_like(flat)
    back = torch.empty_like(flat)
    st = _lib.stream_of(torch.device(DEV))
    _lib.check(L.aq_tile_codes(flat.data_ptr(), N, K, tiled.data_ptr(), st), "tile")
    _lib.check(L.aq_untile_codes(tiled.data_ptr(), N, K, back.data_ptr(), st), "untile")
    assert np.array_equal(tiled.cpu().numpy(), tile_np(flat.cpu().numpy(), N, K))
    assert torch.equal(back, flat)


@pytest.mark.parametrize("M", [1, 5, 16, 40])
def test_grouped_launch_matches_single_calls(M):
    rng = np.random.default_rng(M)
    K = 1024
    ws = [make_weights(rng, (N, K)) for N in (512, 128, 128)]
    qts = [AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=-1) for w in ws]
    bias = [None, torch.from_numpy(rng.standard_normal(128).astype(np.float16)).to(DEV), None]
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).to(DEV)
    ys = AW.qlinear_grouped(x, qts, bias)
    for q, w, b, y in zip(qts, ws, bias, ys):
        w_deq = oref(q, w)
        assert_close(y, reference_linear(x, w_deq, b), x, w_deq)
        assert torch.allclose(y, AW.QuantizedLinear(q, b)(x), rtol=2e-3, atol=1e-3)


def test_int8_weights_run_through_tiled_kernels():
    """int8 (reference format) weights are expanded and tiled once for the
    fused kernels; the result matches F.linear on the dequantized weight."""
    rng = np.random.default_rng(8)
    w = make_weights(rng, (256, 512))
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=128, code_format="int8")
    assert q.code_layout == "flat"
    x = torch.from_numpy(rng.standard_normal((3, 512)).astype(np.float16)).to(DEV)
    w_deq = oref(q, w)
    assert_close(AW.QuantizedLinear(q, None)(x), reference_linear(x, w_deq, None), x, w_deq)
