"""The C ABI: the library loads, exports every function include/atlasinfer_amd.h
declares, reports its ABI version, and rejects bad arguments with a status
code and a message -- all without touching a GPU."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "atlasinfer_amd.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(aq_[a-z0-9_]+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    from atlasinfer_amd import _lib
    return _lib.load()


def test_header_declares_the_expected_api():
    names = declared_functions()
    for must in ["aq_abi_version", "aq_last_error", "aq_quantize", "aq_quantize_finish", "aq_dequantize",
                 "aq_qlinear", "aq_zscore", "aq_compact_codes", "aq_expand_codes", "aq_segment_offsets",
                 "aq_outlier_tiles", "aq_quantize_finish_tiles", "aq_quantize_finish_tiles_grouped"]:
        assert must in names


def test_every_declared_symbol_is_exported(lib):
    from atlasinfer_amd import _lib
    so = _lib.LIB_PATH
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\b(aq_[a-z0-9_]+)\b", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing
    # and the ctypes table covers the header exactly
    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_abi_version(lib):
    from atlasinfer_amd import _lib
    assert lib.aq_abi_version() == _lib.ABI_VERSION
    hdr = open(HEADER).read()
    assert f"#define AQ_ABI_VERSION {_lib.ABI_VERSION}" in hdr


def test_bad_arguments_return_einval_with_message(lib):
    AQ_EINVAL = -1
    p = ctypes.c_void_p(16)
    assert lib.aq_quantize(p, 0, 128, 0x4200, 1, 128, 0, p, p, p, p, 1 << 20, None) == AQ_EINVAL
    assert b"numel" in lib.aq_last_error()
    assert lib.aq_quantize(p, 100, 0, 0x4200, 1, 100, 0, p, p, p, p, 1 << 20, None) == AQ_EINVAL
    assert lib.aq_quantize(p, 100, 1 << 20, 0x4200, 1, 100, 0, p, p, p, p, 1 << 20, None) == AQ_EINVAL
    assert lib.aq_quantize(p, 100, 64, 0x4200, 7, 100, 0, p, p, p, p, 1 << 20, None) == AQ_EINVAL
    assert b"format" in lib.aq_last_error()
    # the tiled layout needs whole 16 x 128 tiles
    assert lib.aq_quantize(p, 100 * 128, 128, 0x4200, 1, 128, 1, p, p, p, p, 1 << 30, None) == AQ_EINVAL
    assert b"tiled" in lib.aq_last_error()
    # G must be a multiple of 32 dividing K for the fused linear
    assert lib.aq_qlinear(p, 1, 4096, 16, p, p, 100, 1, p, p, p, None, None, 0, None, p, p, 1 << 20, None) == AQ_EINVAL
    assert b"block size" in lib.aq_last_error()
    assert lib.aq_qlinear(p, 1, 4000, 16, p, p, 100, 1, p, p, p, None, None, 0, None, p, p, 1 << 20, None) == AQ_EINVAL
    assert b"multiple of 128" in lib.aq_last_error()
    # the dequant-GEMM (M > 64) needs the outlier block lists
    assert lib.aq_qlinear(p, 100, 4096, 16, p, p, 4096, 1, p, p, p, None, None, 0, None, p, p, 0, None) == AQ_EINVAL
    assert b"aq_outlier_tiles" in lib.aq_last_error()
    assert lib.aq_outlier_tiles(p, p, p, 20, 128, p, p, None, None) == AQ_EINVAL
    assert lib.aq_outlier_tiles(p, p, p, 32, 100, p, p, None, None) == AQ_EINVAL
    # the fused finish needs rows of a multiple of 64, blocks tiling them, 16-row tiles
    ws = 1 << 30
    assert lib.aq_quantize_finish_tiles(16 * 100, 100, 100, p, 0, p, ws, p, p, p, p, p, None, None) == AQ_EINVAL
    assert b"aq_quantize_finish_tiles" in lib.aq_last_error()
    assert lib.aq_quantize_finish_tiles(16 * 128, 96, 128, p, 0, p, ws, p, p, p, p, p, None, None) == AQ_EINVAL
    assert lib.aq_quantize_finish_tiles(20 * 128, 128, 128, p, 0, p, ws, p, p, p, p, p, None, None) == AQ_EINVAL
    assert lib.aq_quantize_finish_tiles(16 * 128, 128, 128, p, 5, p, ws, p, p, None, p, p, None, None) == AQ_EINVAL
    assert b"null pointer" in lib.aq_last_error()
    arr = lambda *v: (ctypes.c_int64 * len(v))(*v)  # noqa: E731
    ptrs = (ctypes.c_void_p * 1)(16)
    assert lib.aq_quantize_finish_tiles_grouped(0, arr(2048), 128, 128, ptrs, arr(0), ptrs, arr(ws), ptrs, ptrs,
                                                ptrs, ptrs, ptrs, None, None) == AQ_EINVAL
    assert b"aq_quantize_finish_tiles_grouped" in lib.aq_last_error()
    assert lib.aq_quantize_finish_tiles_grouped(9, arr(2048), 128, 128, ptrs, arr(0), ptrs, arr(ws), ptrs, ptrs,
                                                ptrs, ptrs, ptrs, None, None) == AQ_EINVAL
    assert lib.aq_quantize_finish_tiles_grouped(1, arr(20 * 128), 128, 128, ptrs, arr(0), ptrs, arr(ws), ptrs, ptrs,
                                                ptrs, ptrs, ptrs, None, None) == AQ_EINVAL
    assert lib.aq_dequantize(p, p, 10, 0, 0, 10, 0, None, None, 0, p, None) == AQ_EINVAL
    assert lib.aq_zscore(p, 0, 1e-6, p, None, None) == AQ_EINVAL
    assert lib.aq_tile_codes(p, 20, 128, p, None) == AQ_EINVAL


def test_workspace_sizes(lib):
    assert lib.aq_quantize_workspace_size(4096 * 4096, 4096) >= 4096 * 4096 * 6
    assert lib.aq_quantize_workspace_size(0, 128) == 0
    assert lib.aq_qlinear_workspace_size(1, 4096, 4096) == 0  # the GEMV needs none
    assert lib.aq_qlinear_workspace_size(32, 4096, 4096) == 0
    assert lib.aq_qlinear_workspace_size(64, 14336, 4096) == 0  # tall grid: the GEMV even at M = 64
    assert lib.aq_qlinear_workspace_size(64, 4096, 14336) > 0   # short grid: the GEMM, split K
    # the GEMM on 256 CUs (the count assumed without a device): k_proj's 64
    # tiles of 256 x 128 split K four ways and down_proj's 128 tiles of
    # 256 x 256 two ways, fp32 partial sums of every part; grids that fill
    # the GPU unsplit need none
    assert lib.aq_qlinear_workspace_size(2048, 1024, 4096) == 4 * 2048 * 1024 * 4
    assert lib.aq_qlinear_workspace_size(2048, 4096, 14336) == 2 * 2048 * 4096 * 4
    assert lib.aq_qlinear_workspace_size(2048, 14336, 4096) == 0
    assert lib.aq_max_block_size() == 65536


def test_workspace_too_small_is_reported(lib):
    AQ_EWORKSPACE = -4
    p = ctypes.c_void_p(16)
    assert lib.aq_quantize(p, 4096, 128, 0x4200, 1, 128, 0, p, p, p, p, 16, None) == AQ_EWORKSPACE
    assert b"workspace" in lib.aq_last_error()


def integration_stub():
    """The python block of INTEGRATION.md's reference-side binding section."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    sec = text[text.index("## 3. The reference-side binding"):]
    m = re.search(r"```python\n(.*?)```", sec, flags=re.S)
    assert m, "no python block in the binding section"
    return m.group(1)


def test_integration_stub_binds_the_built_library(lib):
    """The documented ctypes binding, executed as written against the built
    library (no GPU call is made: only argtypes and the ABI assert run), and
    every argtypes list it sets equal to the header's signature."""
    from atlasinfer_amd import _lib
    src = integration_stub().replace('ctypes.CDLL("libatlasinfer_amd.so")', f"ctypes.CDLL({_lib.LIB_PATH!r})")
    ns = {}
    exec(compile(src, "INTEGRATION.md", "exec"), ns)
    so = ns["_so"]
    bound = re.findall(r"_so\.(aq_[a-z0-9_]+)\.argtypes", src)
    assert len(bound) >= 8
    for name in bound:
        want = _lib.SIGNATURES[name][1]
        got = getattr(so, name).argtypes
        assert [t.__name__ for t in got] == [t.__name__ for t in want], name
