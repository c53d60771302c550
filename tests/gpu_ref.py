"""Shared helpers of the GPU tests (not a test module).

The reference weight of every quantized-linear test comes from the CPU oracle
(oracle/aq_oracle.c), never from this library's own dequantize kernel: the
GPU's quantized tensor is first checked bit for bit against the oracle's
codes, scales and outlier lists (codes brought back to element order with
numpy reshapes, not the library's untile kernel, so a tiled-addressing bug
shared by the quantize and linear kernels cannot cancel out), and the
oracle's dequantized weight is then the F.linear operand the layer output is
compared with (the reference's forward is F.linear(x, dequantize_tensor(W),
b), integration/atlas_wrappers.py:56,67).

Tolerance (north star): max|dy| <= 2e-3 max|x| max|w| (plus one fp16 ulp
of the result: the output rounding, see north_star_abs_bound) and rel-L2 <=
1e-3 against the float64 product, plus a per-element bound of one fp16 ulp of
the exact result and the worst-case fp32 accumulation error 2^-20 sum|x||w|.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

DEV = "cuda:0"


def bits(t):
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu()
        return t.view(torch.uint8).numpy() if t.element_size() == 1 else t.view(torch.int16).numpy().view(np.uint16)
    return t.view(np.uint8) if t.dtype.itemsize == 1 else t.view(np.uint16)


def tile_np(flat_codes, N, K):
    """The tiled code layout restated with numpy reshapes: element (n, k) with
    n = 16 rb + r, k = 128 c + 64 h + 16 g + e goes to tile (rb, c), byte
    h*1024 + g*256 + r*16 + e."""
    a = np.asarray(flat_codes, np.uint8).reshape(N // 16, 16, K // 128, 2, 4, 16)  # rb r c h g e
    return np.ascontiguousarray(a.transpose(0, 2, 3, 4, 1, 5)).reshape(-1)


def untile_np(tiled_codes, N, K):
    """Inverse of tile_np."""
    a = np.asarray(tiled_codes, np.uint8).reshape(N // 16, K // 128, 2, 4, 16, 16)  # rb c h g r e
    return np.ascontiguousarray(a.transpose(0, 4, 1, 2, 3, 5)).reshape(-1)


def make_weights(rng, shape, sigma=0.02, frac=0.001, t_dof=None):
    """fp16 weights N(0, sigma) (or Student-t(t_dof) * sigma) with round(frac
    * numel) entries at distinct positions replaced by +-U(8, 20) * sigma
    (the BASELINE weight recipe)."""
    n = int(np.prod(shape))
    w = rng.standard_t(t_dof, n) * sigma if t_dof else rng.standard_normal(n) * sigma
    k = int(round(frac * n))
    pos = rng.permutation(n)[:k]
    w[pos] = rng.choice([-1.0, 1.0], k) * rng.uniform(8, 20, k) * sigma
    return w.reshape(shape).astype(np.float16)


def gpu_dense_codes_np(q, N, K):
    """The GPU tensor's codes, one byte per element of the padded tensor in
    element order, computed on the host: the int8 compacted stream expanded
    at the non-outlier positions, tiled codes untiled with numpy."""
    G = q.block_size
    padded = -(-N * K // G) * G
    raw = bits(q.fp8_data)
    if q.code_format == "int8":
        return O.dense_codes_from_compact(raw, q.outlier_indices.cpu().numpy(), padded)
    if q.code_layout == "tiled":
        return untile_np(raw, N, K)
    return raw


def assert_matches_oracle(q, w, G, fmt, rows=None, thr=3.0):
    """Bit-exact check of GPU QuantizedTensor ``q`` of fp16 array ``w`` [N, K]
    against the oracle: every row, or the listed ``rows`` (blocks must not
    straddle rows then: K % G == 0).  Returns the oracle's result dict for the
    checked rows."""
    N, K = w.shape
    ofmt = O.FMT_INT8 if fmt == "int8" else O.FMT_E4M3
    scales = bits(q.scale_factors)
    idx = q.outlier_indices.cpu().numpy()
    vals = bits(q.fp16_outliers)
    if rows is not None and q.code_layout == "tiled":
        # only the tile rows holding the checked rows leave the device: tile
        # row rb is the contiguous byte range [rb, rb + 1) * 16 K
        rbs = sorted({int(r) // 16 for r in rows})
        dense = np.zeros(N * K, np.uint8)
        for rb in rbs:
            part = bits(q.fp8_data[rb * 16 * K:(rb + 1) * 16 * K])
            dense[rb * 16 * K:(rb + 1) * 16 * K] = untile_np(part, 16, K)
    else:
        dense = gpu_dense_codes_np(q, N, K)
    if rows is None:
        ref = O.quantize(w, G, thr, ofmt)
        assert np.array_equal(scales, bits(ref["scale_factors"])), "scales"
        assert np.array_equal(idx, ref["outlier_indices"]), "outlier indices"
        assert np.array_equal(vals, bits(ref["fp16_outliers"])), "outlier values"
        assert np.array_equal(dense, ref["codes"]), "codes"
        return ref
    assert K % G == 0
    rows = np.asarray(sorted(set(int(r) for r in rows)), np.int64)
    ref = O.quantize(np.ascontiguousarray(w[rows]), G, thr, ofmt)
    bpr = K // G
    sel = (rows[:, None] * bpr + np.arange(bpr)[None, :]).reshape(-1)
    assert np.array_equal(scales[sel], bits(ref["scale_factors"])), "scales (rows)"
    assert np.array_equal(dense.reshape(-1, K)[rows].reshape(-1), ref["codes"]), "codes (rows)"
    row_of = idx // K
    keep = np.isin(row_of, rows)
    remap = np.searchsorted(rows, row_of[keep]) * K + idx[keep] % K
    assert np.array_equal(remap, ref["outlier_indices"]), "outlier indices (rows)"
    assert np.array_equal(vals[keep], bits(ref["fp16_outliers"])), "outlier values (rows)"
    return ref


def oracle_reference(q, w, G, fmt, device=DEV, thr=3.0):
    """Check ``q`` against the oracle over all of ``w`` and return the
    oracle's dequantized weight (fp16, [N, K]) on ``device``."""
    ref = assert_matches_oracle(q, w, G, fmt, thr=thr)
    return torch.from_numpy(O.dequantize(ref)).to(device)


def untile_torch(tiled, N, K):
    """untile_np with torch reshapes (on the tensor's own device)."""
    a = tiled.view(torch.uint8).reshape(N // 16, K // 128, 2, 4, 16, 16)  # rb c h g r e
    return a.permute(0, 4, 1, 2, 3, 5).contiguous().reshape(-1)


def torch_dequant(q, N, K, device=DEV):
    """dequantize_tensor restated with torch ops from q's fields (codes in
    element order by reshapes, torch's own float8_e4m3fn / int8 conversions,
    one f32 product per element rounded once to fp16, outliers written
    back): the reference weight for large models whose quantized tensors are
    checked against the oracle on row slices only (assert_matches_oracle
    with ``rows``)."""
    G = q.block_size
    if q.code_format == "e4m3" and q.code_layout == "tiled":
        dense = untile_torch(q.fp8_data.to(device), N, K)
    else:
        dense = torch.from_numpy(gpu_dense_codes_np(q, N, K)).to(device)
    if q.code_format == "int8":
        v = dense.view(torch.int8).float()
    else:
        v = dense.view(torch.float8_e4m3fn).float()
    s = q.scale_factors.to(device).float().repeat_interleave(G)
    w = (v * s)[: N * K].half()
    idx = q.outlier_indices.to(device)
    inside = idx < N * K
    w[idx[inside]] = q.fp16_outliers.to(device)[inside]
    return w.view(N, K)


def reference_linear(x, w_ref, bias):
    y = x.double() @ w_ref.double().t()
    if bias is not None:
        y = y + bias.double()
    return y


def fp16_ulp(v):
    a = v.abs().clamp(min=2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 10)


def north_star_abs_bound(yref, x, w):
    """Per-element form of the north-star max-abs bound used here:
    2e-3 max|x| max|w| plus one fp16 ulp of the exact result.  The ulp term
    is the output rounding every fp16-output linear incurs, the reference's
    own F.linear included: half an ulp of |y| exceeds 2e-3 max|x| max|w|
    alone once |y| > 4 max|x| max|w| (e.g. outlier-free layers with a few
    thousand inputs), where no fp16 result can meet the bound without it
    (test_gpu_configs.py::test_literal_bound_misses_fp16_output_rounding
    shows torch's F.linear missing it on such inputs)."""
    return 2e-3 * x.abs().max().double() * w.abs().max().double() + fp16_ulp(yref)


def assert_close(y, yref, x, w):
    """North-star tolerance (max-abs with the output-rounding term, see
    north_star_abs_bound; rel-L2 <= 1e-3), plus a per-element bound: one
    fp16 ulp of the exact result (the output rounding) plus the worst-case
    fp32 accumulation error over the row, 2^-20 * sum_k |x_k| |w_nk|."""
    d = (y.double() - yref).abs()
    excess = (d / north_star_abs_bound(yref, x, w)).max().item()
    assert excess <= 1.0, excess
    rel = (y.double() - yref).norm() / yref.norm()
    assert rel <= 1e-3, rel.item()
    x2 = x.reshape(-1, x.shape[-1]).double().abs()
    acc = (x2 @ w.double().abs().t()).reshape(yref.shape)
    strict = fp16_ulp(yref) + 2.0 ** -20 * acc
    worst = (d / strict).max().item()
    assert worst <= 1.0, worst
