"""CPU checks that pin the oracle (oracle/aq_oracle.c) before it is trusted.

* golden vectors written by the reference itself (tests/golden/make_golden.py)
  -- bit-exact codes, scales, outlier lists, dequantized tensors, z-scores;
* the fp16 and E4M3 conversions against numpy / torch over every fp16 input;
* closed-form properties a plausible slip (wrong rounding, dropped clamp,
  off-by-one in padding, swapped operands) would break.
"""
import os
import subprocess

import numpy as np
import pytest
import torch

from conftest import GOLDEN_DIR, ROOT, golden_cases

CASES = golden_cases()


@pytest.mark.parametrize("name,d", CASES, ids=[c[0] for c in CASES])
def test_oracle_matches_reference_golden(oracle, name, d):
    q = oracle.quantize(d["x"], int(d["block_size"]), float(d["z_threshold"]), oracle.FMT_INT8)
    assert np.array_equal(q["fp8_data"].view(np.uint8), d["fp8_data"].view(np.uint8))
    assert np.array_equal(q["scale_factors"].view(np.uint16), d["scale_factors"].view(np.uint16))
    assert np.array_equal(q["outlier_indices"], d["outlier_indices"])
    assert np.array_equal(q["fp16_outliers"].view(np.uint16), d["fp16_outliers"].view(np.uint16))
    deq = oracle.dequantize(q)
    assert np.array_equal(deq.view(np.uint16), d["deq"].view(np.uint16))
    # the reference's own layout (compacted stream) dequantizes identically
    q2 = {k: v for k, v in q.items() if k != "codes"}
    assert np.array_equal(oracle.dequantize(q2).view(np.uint16), d["deq"].view(np.uint16))


def test_oracle_zscore_matches_reference_golden(oracle):
    with np.load(os.path.join(GOLDEN_DIR, "zscore.npz")) as d:
        off = 0
        for n in d["lens"]:
            z, _ = oracle.zscore(d["x"][off:off + n])
            assert np.array_equal(z.view(np.uint16), d["z"][off:off + n].view(np.uint16)), n
            off += n


def test_f2h_matches_numpy_on_all_fp16_and_neighbours(oracle):
    L = oracle.lib()
    rng = np.random.default_rng(0)
    # every fp16 value, the midpoints between neighbours, and random f32
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    f = h.astype(np.float32)
    fin = np.isfinite(f)
    mids = ((f[fin][:-1].astype(np.float64) + f[fin][1:]) / 2).astype(np.float32)
    rand = rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 5, 20000)
    vals = np.concatenate([f[fin], mids, np.nextafter(mids, np.float32(np.inf)),
                           np.nextafter(mids, np.float32(-np.inf)), rand]).astype(np.float32)
    ours = np.array([L.aqo_f2h(float(v)) for v in vals[::7]], np.uint16)
    ref = vals[::7].astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_e4m3_encoding_matches_torch_over_all_fp16(oracle):
    ours = oracle.e4m3_encode_all_f16()
    h = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.float16)
    finite = torch.isfinite(h)
    ref = h.float().clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours[finite.numpy()], ref[finite.numpy()])


def test_e4m3_decode_is_exact_inverse(oracle):
    L = oracle.lib()
    for c in range(256):
        if (c & 0x7F) == 0x7F:
            continue
        v = L.aqo_e4m3_to_double(c)
        assert L.aqo_e4m3_encode(v) == c or (v == 0 and (c & 0x7F) == 0)
        assert v == torch.tensor([c], dtype=torch.uint8).view(torch.float8_e4m3fn).double().item()


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("G", [8, 100, 128, 1024])
def test_quantize_error_bounds(oracle, fmt, G):
    """|x - deq| bounded by the code grid: int8 <= 0.5625 s (0.5 from integer
    rounding, 127 * 2^-11 from the fp16 quotient) plus the fp16 rounding of
    the product; e4m3 relative error <= 2^-4 (+ the same fp16 terms)."""
    rng = np.random.default_rng(G + 7 * fmt)
    w = (rng.standard_normal(8 * 1024) * 0.02).astype(np.float16)
    q = oracle.quantize(w, G, 3.0, fmt)
    deq = oracle.dequantize(q).astype(np.float64)
    x = w.astype(np.float64)
    s = np.repeat(q["scale_factors"].astype(np.float64), G)[: x.size]
    inl = ~q["is_outlier"][: x.size].astype(bool)
    err = np.abs(x - deq)[inl]
    if fmt == 0:
        assert np.all(err <= 0.5625 * s[inl] + np.abs(x[inl]) * 2.0 ** -10 + 2.0 ** -24)
        assert np.all(np.abs(q["codes"].view(np.int8)) <= 127)
    else:
        tiny = 2.0 ** -9 * s[inl]  # E4M3 subnormal spacing
        assert np.all(err <= np.abs(x[inl]) * (2.0 ** -4 + 2.0 ** -9) + tiny + 2.0 ** -24)
    # outliers come back verbatim
    out = q["is_outlier"][: x.size].astype(bool)
    assert np.array_equal(deq[out], x[out])


def test_outlier_count_respects_sample_bound(oracle):
    """sum z^2 = G - 1 for sample z-scores, so at most (G-1)/thr^2 elements of
    a block can exceed thr (up to fp16 rounding of mean/std)."""
    rng = np.random.default_rng(3)
    for G, thr in [(128, 3.0), (4096, 3.0), (64, 2.0)]:
        w = rng.standard_t(2, size=64 * G).astype(np.float16)
        q = oracle.quantize(w, G, thr, 0)
        per_block = q["is_outlier"].reshape(-1, G).sum(1)
        assert per_block.max() <= (G - 1) / thr ** 2 + 1


def test_padding_and_small_blocks(oracle):
    """numel not a multiple of G: the tail is zero-padded, codes exist for the
    padding, outliers in the padding are kept in the index list."""
    w = np.full(10, 0.5, np.float16)
    w[3] = 8.0
    q = oracle.quantize(w, 64, 3.0, 0)
    assert q["scale_factors"].size == 1
    assert q["fp8_data"].size + q["outlier_indices"].size == 64
    assert oracle.dequantize(q).shape == (10,)


def test_constant_and_zero_blocks(oracle):
    """std = 0: den = fp16(1e-6); a constant block has no outliers and codes
    of +-127 (int8) or +-448 (e4m3); a zero block has scale fp16(1e-6)."""
    w = np.concatenate([np.full(64, 0.25, np.float16), np.zeros(64, np.float16)])
    for fmt, top in [(0, 127), (1, 448)]:
        q = oracle.quantize(w, 64, 3.0, fmt)
        assert q["outlier_indices"].size == 0
        s = q["scale_factors"]
        assert s[1] == np.float16(1e-6)
        assert np.float16(s[0]) == np.float16(np.float32(0.25) / np.float32(top))


def test_brute_force_tiny_blocks_against_float64(oracle):
    """For tiny blocks every step can be recomputed directly: mean/std from
    numpy float64, the z test, scale and codes; compare element by element."""
    rng = np.random.default_rng(11)
    for trial in range(200):
        G = int(rng.integers(2, 9))
        w = (rng.standard_normal(G) * rng.choice([0.02, 1.0, 50.0])).astype(np.float16)
        if trial % 5 == 0:
            w[rng.integers(0, G)] *= 40
        q = oracle.quantize(w, G, 1.5, 0)
        x = w.astype(np.float64)
        mean = np.float16(np.float32(x.mean()))
        std = np.float16(np.float32(x.std(ddof=1)))
        den = np.float16(np.float32(std) + np.float32(1e-6))
        d = (w.astype(np.float32) - np.float32(mean)).astype(np.float16)
        z = (d.astype(np.float32) / np.float32(den)).astype(np.float16)
        out = np.abs(z) > np.float16(1.5)
        assert np.array_equal(out, q["is_outlier"].astype(bool)), (w, z)
        inl = ~out
        if inl.any():
            amax = np.abs(w[inl]).max()
            s = np.float16(np.float32(amax) / np.float32(127.0))
            s = max(s, np.float16(1e-6))
            assert q["scale_factors"][0] == s
            qq = (w[inl].astype(np.float32) / np.float32(s)).astype(np.float16)
            codes = np.clip(np.rint(qq.astype(np.float32)), -127, 127).astype(np.int8)
            assert np.array_equal(codes, q["fp8_data"])


def test_kernel_arithmetic_identities():
    """The quantize kernel replaces literal divisions by cheaper forms; check
    the identities against the literal arithmetic: the Newton-corrected and
    the single fused-product quotients for every fp16 x and every 16th
    positive fp16 scale (every scale: `c_kernel_math_check 1`, about 3e9
    pairs, run during development with 0 differences), and the outlier cut
    for 100 random dens x 9 thresholds x every fp16 |x - mean|."""
    build = os.path.join(ROOT, "oracle", "_build")
    os.makedirs(build, exist_ok=True)
    exe = os.path.join(build, "c_kernel_math_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, os.path.join(ROOT, "tests", "c_kernel_math_check.c"),
                    os.path.join(ROOT, "oracle", "aq_oracle.c"), "-lm"], check=True)
    r = subprocess.run([exe, "16", "100"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "quotient:" in r.stdout and "product:" in r.stdout and "threshold:" in r.stdout, r.stdout
    for line in r.stdout.splitlines():
        assert " 0 code differences" in line or line.startswith("threshold"), line
    assert "0 normal-quotient differences" in r.stdout and "pairs, 0 differences" in r.stdout, r.stdout
