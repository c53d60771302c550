"""aq_qlinear_noalloc (no workspace argument; split-K partial sums in the
library's static device array) against aq_qlinear given a caller workspace of
the same size: bit-identical outputs (same plan, same kernels), on two calls
in a row, the second with a smaller input, and both within the north-star
bounds of F.linear on the oracle's weight.  Through the C ABI."""
import numpy as np
import pytest
import torch

import gpu_ref as R
from atlasinfer_amd import _lib
from atlasinfer_core.quant import adaptive_quantizer as AQ

pytestmark = pytest.mark.gpu
DEV = R.DEV


def _weight(seed, N, K):
    w = R.make_weights(np.random.default_rng(seed), (N, K))
    q = AQ.quantize_tensor(torch.from_numpy(w).to(DEV), block_size=-1, code_format="e4m3")
    return q, R.oracle_reference(q, w, K, "e4m3")


def _call(fn, q, x, bias, *ws):
    L = _lib.load()
    dev = torch.device(DEV)
    K = int(q.original_shape[-1])
    N = q.original_shape.numel() // K
    M = x.shape[0]
    codes = AQ.kernel_codes(q, dev)
    tp, te, tmax = AQ.outlier_tiles(q, dev)
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV)
    _lib.check(getattr(L, fn)(x.data_ptr(), M, K, N, codes.data_ptr(), q.scale_factors.data_ptr(), q.block_size,
                              _lib.FMT_E4M3, q.outlier_row_ptr.data_ptr(), _lib.ptr(q.outlier_cols),
                              _lib.ptr(q.fp16_outliers), tp.data_ptr(), te.data_ptr(), tmax, _lib.ptr(bias),
                              y.data_ptr(), *ws, _lib.stream_of(dev)), fn)
    return y


def test_noalloc_matches_workspace_entry_point():
    ws = torch.empty(_lib.NOALLOC_SCRATCH_BYTES, dtype=torch.uint8, device=DEV)
    # first call: down_proj at M = 2048 (split two ways: 64 MiB of partial
    # sums, the whole scratch); second: k_proj-sized at M = 512 (a smaller
    # input, split four ways), then a decode-sized call (no scratch used)
    for seed, (M, N, K) in enumerate([(2048, 4096, 14336), (512, 1024, 4096), (1, 1024, 4096)]):
        q, w_ref = _weight(seed, N, K)
        x = torch.from_numpy(np.random.default_rng(100 + seed).standard_normal((M, K)).astype(np.float16)).to(DEV)
        bias = torch.from_numpy((np.random.default_rng(200 + seed).standard_normal(N) * 0.1)
                                .astype(np.float16)).to(DEV)
        y0 = _call("aq_qlinear_noalloc", q, x, bias)
        y1 = _call("aq_qlinear", q, x, bias, ws.data_ptr(), ws.numel())
        torch.cuda.synchronize()
        assert torch.equal(y0, y1), (M, N, K)
        R.assert_close(y0, R.reference_linear(x, w_ref, bias), x, w_ref)
