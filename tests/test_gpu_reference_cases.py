"""The reference's own quantizer test (/root/reference/tests/test_quantizer.py:
13-56), replayed through the drop-in API (atlasinfer_core.quant.
adaptive_quantizer, the same import path the reference test uses).

* code_format="int8" (the reference's format) must pass the reference's
  assertions as written: reconstruction MSE < 1e-3 on randn * 5 with every
  150th element x10 at block 64, z = 3.5 (:13-40), MSE < 1e-3 on a tensor
  smaller than one block (:42-49), and an empty tensor that round-trips its
  shape (:51-56); the memoised second dequantize returns the same tensor.
* code_format="e4m3" (this build's default storage format) keeps 3 mantissa
  bits instead of int8's 254 uniform steps, so its MSE on case 1 is about
  16x higher and does NOT meet the reference's 1e-3: the test records it and
  checks it against E4M3's own closed-form bound instead (each non-outlier
  reconstructed within 2^-4 of its value relative, or the E4M3 subnormal
  step 2^-9 s absolute, plus one fp16 rounding).
"""
import numpy as np
import pytest
import torch

from atlasinfer_core.quant.adaptive_quantizer import (QuantizedTensor, clear_dequantized_cache, dequantize_tensor,
                                                      quantize_tensor)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case1_tensor():
    torch.manual_seed(0)
    t = (torch.randn(128, 256, dtype=torch.float32) * 5).to(torch.float16).to(DEV)
    t.view(-1)[::150] *= 10
    return t


@pytest.mark.parametrize("fmt", ["int8", "e4m3"])
def test_reference_case1_standard(fmt):
    original = case1_tensor()
    q = quantize_tensor(original.cpu(), block_size=64, z_threshold=3.5, code_format=fmt)
    assert isinstance(q, QuantizedTensor)
    assert q.fp8_data.device.type == "cpu"  # results on the input's device, as the reference returns them
    assert q.memory_footprint() < original.element_size() * original.nelement()
    clear_dequantized_cache()
    rec = dequantize_tensor(q, target_device=DEV)
    assert dequantize_tensor(q, target_device=DEV) is rec  # the memoised tensor
    mse = torch.mean(torch.abs(original - rec).float() ** 2).item()
    print(f"{fmt}: reconstruction MSE {mse:.6f}, outliers {q.fp16_outliers.numel()}")
    if fmt == "int8":
        assert mse < 1e-3, mse  # the reference's assertion (test_quantizer.py:40)
    else:
        # E4M3: per-element bound against the block scale s of each element
        o = original.double().view(-1)
        r = rec.double().view(-1)
        s = q.scale_factors.to(DEV).double().repeat_interleave(64)[: o.numel()]
        out = torch.zeros_like(o, dtype=torch.bool)
        out[q.outlier_indices.to(DEV)] = True
        err = (o - r).abs()
        bound = torch.maximum(o.abs() * 2.0 ** -4, s * 2.0 ** -9) + o.abs() * 2.0 ** -10 + s * 2.0 ** -10
        assert torch.all(err[out] == 0)
        assert torch.all(err[~out] <= bound[~out])
        assert 1e-3 < mse < 0.05, mse  # the stated difference from the reference's 1e-3
    clear_dequantized_cache()


@pytest.mark.parametrize("fmt", ["int8", "e4m3"])
def test_reference_case2_small_and_case3_empty(fmt):
    torch.manual_seed(1)
    small = torch.randn(10, dtype=torch.float16).to(DEV)
    q = quantize_tensor(small.cpu(), block_size=64, code_format=fmt)
    rec = dequantize_tensor(q, target_device=DEV)
    mse = torch.mean((small - rec).float() ** 2).item()
    assert mse < 1e-3, mse  # test_quantizer.py:49
    empty = torch.empty((0, 10), dtype=torch.float16).to(DEV)
    qe = quantize_tensor(empty.cpu(), code_format=fmt)
    assert dequantize_tensor(qe, target_device=DEV).shape == empty.shape  # :56
    clear_dequantized_cache()
