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


def test_caller_stream_order():
    """quantize_tensors on a caller's stream, its inputs written on that
    stream just before the call (behind a long matmul) and its outputs read
    on it just after, with no synchronisation in between: the call's kernels
    follow the caller's earlier work and precede its later work."""
    shapes = [(4096, 4096), (1024, 14336), (2048, 4096), (512, 14336)]
    base = [_w(s, 70 + i) for i, s in enumerate(shapes)]
    ref = [AQ.quantize_tensor(w, block_size=-1, code_format="e4m3") for w in base]
    ws = [torch.zeros_like(w) for w in base]
    a = torch.randn(8192, 8192, device=DEV, dtype=torch.float16)
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=DEV)
    with torch.cuda.stream(s):
        for _ in range(4):
            a = torch.matmul(a, a) * 1e-3
        for w, b in zip(ws, base):
            w.copy_(b)
        qs = AQ.quantize_tensors(ws, block_size=-1, code_format="e4m3")
        got = [[None if getattr(q, f) is None else getattr(q, f).clone() for f in FIELDS] for q in qs]
    torch.cuda.synchronize()
    for q, r, g in zip(qs, ref, got):
        for f, t in zip(FIELDS, g):
            x = getattr(r, f)
            if x is None:
                assert t is None, f
            else:
                assert torch.equal(t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t,
                                   x.view(torch.uint8) if x.dtype == torch.float8_e4m3fn else x), f
        assert int(q.outlier_tile_max) == int(r.outlier_tile_max)


def test_copied_inputs_on_second_stream():
    """Inputs that need a copy first (transposed views, a host tensor) in
    grouped runs: results as quantize_tensor gives them, on the inputs'
    devices."""
    ws = [_w((4096, 4096), 80), _w((14336, 1024), 81).t(), _w((4096, 1024), 82), _w((14336, 512), 83).t()]
    ws[2] = ws[2].cpu()
    got = AQ.quantize_tensors(ws, block_size=-1, code_format="e4m3")
    for w, q in zip(ws, got):
        r = AQ.quantize_tensor(w, block_size=-1, code_format="e4m3")
        _same(q.to(DEV), r.to(DEV))
