"""The CPU baseline's restatement of the reference's per-block loops
(oracle/ref_loop.py, timed by bench.py's cpu_baseline leg) reproduces the
reference's own outputs: every golden fixture (written by the reference's
quantize_tensor / dequantize_tensor, tests/golden/make_golden.py) bit for
bit, so the timed loop is the reference's computation."""
import numpy as np
import pytest
import torch

from conftest import golden_cases

CASES = golden_cases()


@pytest.mark.parametrize("name,d", CASES, ids=[c[0] for c in CASES])
def test_ref_loops_match_reference_golden(name, d):
    from oracle import ref_loop
    x = torch.from_numpy(d["x"])
    G = int(d["block_size"])
    if x.numel() > 40000:
        pytest.skip("large case: covered by the smaller fixtures (Python loop)")
    codes, outs, idx, scales, nb = ref_loop.quantize_loop(x, G, float(d["z_threshold"]))
    assert np.array_equal(codes.numpy(), d["fp8_data"])
    assert np.array_equal(outs.numpy().view(np.uint16), d["fp16_outliers"].view(np.uint16))
    assert np.array_equal(idx.numpy(), d["outlier_indices"])
    assert np.array_equal(scales.numpy().view(np.uint16), d["scale_factors"].view(np.uint16))
    deq, _ = ref_loop.dequantize_loop(codes, outs, idx, scales, x.numel(), G)
    assert np.array_equal(deq[:x.numel()].numpy().view(np.uint16), d["deq"].reshape(-1).view(np.uint16))
