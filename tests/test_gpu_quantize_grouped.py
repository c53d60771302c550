"""quantize_tensors / aq_quantize_grouped: a layer's weights quantized by
one launch per 8 get exactly what quantize_tensor gives each alone (codes,
scales, outlier values, indices, CSR rows, block lists), whatever mix of
shapes, formats, layouts and group sizes; members too large to group take
the single path in the same call."""
import pytest
import torch

from atlasinfer_amd.quant import adaptive_quantizer as AQ

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
FIELDS = ("fp8_data", "fp16_outliers", "outlier_indices", "scale_factors", "outlier_row_ptr", "outlier_cols",
          "outlier_tile_ptr", "outlier_tile_ent")


def _w(shape, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(*shape, generator=g, device=DEV) * 0.02
    m = torch.rand(*shape, generator=g, device=DEV) < 3e-3
    return torch.where(m, torch.sign(torch.randn(*shape, generator=g, device=DEV)) * 0.3, w).half()


def _same(a, b):
    for f in FIELDS:
        x, y = getattr(a, f), getattr(b, f)
        assert (x is None) == (y is None), f
        if x is not None:
            assert x.dtype == y.dtype and torch.equal(x.view(torch.uint8) if x.dtype == torch.float8_e4m3fn else x,
                                                      y.view(torch.uint8) if y.dtype == torch.float8_e4m3fn else y), f
    assert a.original_shape == b.original_shape and a.block_size == b.block_size and a.code_layout == b.code_layout
    assert int(a.outlier_tile_max) == int(b.outlier_tile_max)


@pytest.mark.parametrize("fmt,bs", [("e4m3", -1), ("e4m3", 128), ("int8", 128)])
def test_grouped_equals_single(fmt, bs):
    shapes = [(1024, 4096), (4096, 4096), (512, 4096), (14336, 4096), (4096, 14336), (2, 64, 4096), (100, 4096),
              (96, 2048)]
    ws = [_w(s, 20 + i) for i, s in enumerate(shapes)]
    grouped = AQ.quantize_tensors(ws, block_size=bs, code_format=fmt)
    for w, q in zip(ws, grouped):
        _same(q, AQ.quantize_tensor(w, block_size=bs, code_format=fmt))


def test_more_members_than_one_launch_takes():
    """Eleven weights of one shape: two launches (8 + 3)."""
    ws = [_w((256, 4096), 40 + i) for i in range(11)]
    for w, q in zip(ws, AQ.quantize_tensors(ws, block_size=-1, code_format="e4m3")):
        _same(q, AQ.quantize_tensor(w, block_size=-1, code_format="e4m3"))


def test_grouped_wide_rows():
    """Rows wider than one workgroup's block-list sort (K = 32768: 512
    chunks of 64): the grouped finish takes each member's two-launch path;
    results as quantize_tensor gives them."""
    ws = [_w((32, 32768), 60 + i) for i in range(3)]
    for w, q in zip(ws, AQ.quantize_tensors(ws, block_size=-1, code_format="e4m3")):
        assert q.outlier_tile_ptr is not None
        _same(q, AQ.quantize_tensor(w, block_size=-1, code_format="e4m3"))
