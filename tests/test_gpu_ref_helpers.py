"""CPU checks of the GPU tests' reference helpers (tests/gpu_ref.py): a
QuantizedTensor built from the oracle's own results (tiled e4m3, flat int8)
passes the bit-exact comparison in full and on row slices, a single flipped
code or scale fails it, and the torch restatement of dequantize_tensor
equals the oracle's dequantize bit for bit."""
import numpy as np
import pytest
import torch

import gpu_ref as R
from atlasinfer_core.quant import adaptive_quantizer as AQ


def qt_like_gpu(oracle, w, G, fmt):
    """What quantize_tensor returns, assembled from the oracle on the host."""
    ref = oracle.quantize(w, G, 3.0, oracle.FMT_INT8 if fmt == "int8" else oracle.FMT_E4M3)
    N, K = w.shape
    if fmt == "int8":
        codes, layout = torch.from_numpy(ref["fp8_data"]), "flat"
    else:
        codes, layout = torch.from_numpy(R.tile_np(ref["codes"], N, K)).view(torch.float8_e4m3fn), "tiled"
    return AQ.QuantizedTensor(codes, torch.from_numpy(ref["fp16_outliers"]), torch.from_numpy(ref["outlier_indices"]),
                              torch.from_numpy(ref["scale_factors"]), torch.Size(w.shape), G, fmt,
                              code_layout=layout)


@pytest.mark.parametrize("fmt,G", [("e4m3", 256), ("e4m3", 64), ("int8", 128)])
def test_helpers_accept_the_oracle_and_reject_a_flip(oracle, fmt, G):
    rng = np.random.default_rng(3)
    w = R.make_weights(rng, (48, 256), frac=0.01, t_dof=3)
    q = qt_like_gpu(oracle, w, G, fmt)
    R.assert_matches_oracle(q, w, G, fmt)
    R.assert_matches_oracle(q, w, G, fmt, rows=[0, 17, 47])
    w_ref = R.oracle_reference(q, w, G, fmt, device="cpu")
    assert np.array_equal(R.bits(R.torch_dequant(q, 48, 256, device="cpu")), R.bits(w_ref))
    # one flipped code bit, found by both the full and the row-slice check
    raw = q.fp8_data.view(torch.uint8).clone()
    pos = int(np.nonzero(R.bits(raw))[0][7])
    raw[pos] ^= 1
    bad = q._replace(fp8_data=raw.view(q.fp8_data.dtype))
    with pytest.raises(AssertionError):
        R.assert_matches_oracle(bad, w, G, fmt)
    row = int(np.nonzero(np.any(R.gpu_dense_codes_np(bad, 48, 256).reshape(48, 256) !=
                                R.gpu_dense_codes_np(q, 48, 256).reshape(48, 256), axis=1))[0][0])
    with pytest.raises(AssertionError):
        R.assert_matches_oracle(bad, w, G, fmt, rows=[row])
    s = q.scale_factors.clone()
    s[3] = s[3] + 1
    with pytest.raises(AssertionError):
        R.assert_matches_oracle(q._replace(scale_factors=s), w, G, fmt)


def test_untile_inverts_tile():
    rng = np.random.default_rng(0)
    a = rng.integers(0, 256, 32 * 384).astype(np.uint8)
    t = R.tile_np(a, 32, 384)
    assert not np.array_equal(t, a)
    assert np.array_equal(R.untile_np(t, 32, 384), a)
    assert np.array_equal(R.untile_torch(torch.from_numpy(t), 32, 384).numpy(), a)
