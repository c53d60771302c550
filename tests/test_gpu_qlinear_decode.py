"""aq_qlinear_decode (the decode GEMVs with a prologue and epilogue) against
the same work done by separate launches: the plain grouped GEMV, torch's
fp16 ReLU / add, aq_silu_mul, and HF's RMSNorm / torch's LayerNorm modules.

Where the fused launch stages the very x the separate launches produce
(no prologue, SwiGLU) its outputs must be bit-identical to theirs; with a
norm prologue the row's statistics are summed in another order than the
norm modules', so the outputs agree to the layer tolerance instead."""
import ctypes

import pytest
import torch

from atlasinfer_amd import _lib
from atlasinfer_amd.integration.atlas_wrappers import (PRO_LAYERNORM, PRO_NONE, PRO_RMS, PRO_SWIGLU,
                                                       qlinear_decode, qlinear_grouped)
from atlasinfer_amd.quant.adaptive_quantizer import kernel_codes, quantize_tensor

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _weights(Ns, K, seed, block_size=-1, code_format="e4m3"):
    g = torch.Generator(device=DEV).manual_seed(seed)
    qts = []
    for N in Ns:
        w = torch.randn(N, K, generator=g, device=DEV) * 0.02
        m = torch.rand(N, K, generator=g, device=DEV) < 1e-3  # 0.1 % outliers
        w = torch.where(m, torch.sign(torch.randn(N, K, generator=g, device=DEV)) * 0.3, w).half()
        qts.append(quantize_tensor(w, block_size=block_size, code_format=code_format))
    return qts


def _close(a, b, what):
    a, b = a.float(), b.float()
    err = (a - b).abs().max().item()
    rel = ((a - b).norm() / b.norm().clamp_min(1e-12)).item()
    assert rel <= 1e-3 and err <= 2e-3 * b.abs().max().item() + 1e-3, (what, err, rel)


@pytest.mark.parametrize("M", [1, 8, 32])
@pytest.mark.parametrize("Ns,K,bs", [([512, 128, 128], 2048, -1), ([2048], 8192, -1), ([4096, 4096], 1024, 128),
                                     ([1024], 4096, 256)])
def test_epilogue_residual_and_relu_bit_exact(Ns, K, bs, M):
    """M = 1 takes the x-in-LDS GEMV, M = 8 and 32 the shared-x GEMV."""
    qts = _weights(Ns, K, 1, bs)
    codes = [kernel_codes(q, DEV) for q in qts]
    g = torch.Generator(device=DEV).manual_seed(2)
    x = torch.randn(M, K, generator=g, device=DEV).half()
    biases = [torch.randn(N, generator=g, device=DEV).half() if i == 0 else None for i, N in enumerate(Ns)]
    res = [torch.randn(M, N, generator=g, device=DEV).half() for N in Ns]
    ref = qlinear_grouped(x, qts, biases, codes)
    out = qlinear_decode(x, qts, biases, codes)
    for a, b in zip(out, ref):
        assert torch.equal(a, b)
    relu = [i % 2 for i in range(len(Ns))]
    out = qlinear_decode(x, qts, biases, codes, residuals=res, relu=relu)
    for a, b, r, act in zip(out, ref, res, relu):
        assert torch.equal(a, (torch.relu(b) if act else b) + r)


@pytest.mark.parametrize("Ns,K,bs", [([2048], 8192, -1), ([14336, 14336], 4096, -1), ([1024], 2048, 128)])
def test_swiglu_prologue_bit_exact(Ns, K, bs):
    """x holds the gate, x2 the up projection: identical to aq_silu_mul
    followed by the plain GEMV, bit for bit."""
    M = 1
    qts = _weights(Ns, K, 3, bs)
    codes = [kernel_codes(q, DEV) for q in qts]
    g = torch.Generator(device=DEV).manual_seed(4)
    gate = (torch.randn(M, K, generator=g, device=DEV) * 3).half()
    up = torch.randn(M, K, generator=g, device=DEV).half()
    a = torch.empty_like(gate)
    _lib.check(_lib.load().aq_silu_mul(gate.data_ptr(), up.data_ptr(), a.data_ptr(), M * K, _lib.stream_of(DEV)),
               "aq_silu_mul")
    ref = qlinear_grouped(a, qts, [None] * len(Ns), codes)
    res = [torch.randn(M, N, generator=g, device=DEV).half() for N in Ns]
    out = qlinear_decode(gate, qts, [None] * len(Ns), codes, PRO_SWIGLU, x2=up, residuals=res)
    for o, b, r in zip(out, ref, res):
        assert torch.equal(o, b + r)


@pytest.mark.parametrize("M", [8, 32, 64])
@pytest.mark.parametrize("N,K,bs", [(14336, 4096, -1), (4096, 1024, 128), (2048, 2048, -1)])
def test_swiglu_pair_epilogue(N, K, bs, M):
    """gate and up in one launch writing fp16(fp16(silu(g)) u): bit for bit
    the same GEMV's two outputs through aq_silu_mul where both take the same
    waves per tile row (a pair takes at most 4: 2048 + 2048 rows at M <= 32
    take 8 alone), else to the layer tolerance."""
    qts = _weights([N, N], K, 11, bs)
    codes = [kernel_codes(q, DEV) for q in qts]
    g = torch.Generator(device=DEV).manual_seed(12)
    x = torch.randn(M, K, generator=g, device=DEV).half()
    biases = [torch.randn(N, generator=g, device=DEV).half() * 0.1 for _ in range(2)]
    gate, up = qlinear_decode(x, qts, biases, codes)
    ref = torch.empty_like(gate)
    _lib.check(_lib.load().aq_silu_mul(gate.data_ptr(), up.data_ptr(), ref.data_ptr(), M * N, _lib.stream_of(DEV)),
               "aq_silu_mul")
    out = qlinear_decode(x, qts, biases, codes, swiglu_pair=True)
    assert len(out) == 1 and out[0].shape == (M, N)
    if N == 2048 and M <= 32:
        _close(out[0], ref, "SwiGLU pair")
    else:
        assert torch.equal(out[0], ref)
    again = qlinear_decode(x, qts, biases, codes, swiglu_pair=True)[0]
    assert torch.equal(again, out[0])  # deterministic


@pytest.mark.parametrize("mode,Ns,K,bs", [(PRO_RMS, [4096, 1024, 1024], 4096, -1), (PRO_RMS, [14336, 14336], 4096, -1),
                                          (PRO_LAYERNORM, [2048, 2048, 2048], 2048, -1),
                                          (PRO_LAYERNORM, [8192], 2048, 128), (PRO_RMS, [12288, 12288], 16384, -1)])
def test_norm_prologue_matches_modules(mode, Ns, K, bs):
    """RMSNorm / LayerNorm folded into the launch against HF's LlamaRMSNorm /
    torch's LayerNorm followed by the plain GEMV ([12288, 12288] x 16384
    stages its row over several rounds with one wave per tile row)."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    qts = _weights(Ns, K, 5, bs)
    codes = [kernel_codes(q, DEV) for q in qts]
    g = torch.Generator(device=DEV).manual_seed(6)
    x = (torch.randn(1, K, generator=g, device=DEV) * 4).half()
    if mode == PRO_RMS:
        norm = LlamaRMSNorm(K, eps=1e-5).to(DEV).half()
        with torch.no_grad():
            norm.weight.copy_((torch.rand(K, generator=g, device=DEV) + 0.5).half())
        nw, nb, eps = norm.weight, None, 1e-5
    else:
        norm = torch.nn.LayerNorm(K).to(DEV).half()
        with torch.no_grad():
            norm.weight.copy_((torch.rand(K, generator=g, device=DEV) + 0.5).half())
            norm.bias.copy_((torch.randn(K, generator=g, device=DEV) * 0.1).half())
        nw, nb, eps = norm.weight, norm.bias, norm.eps
    with torch.no_grad():
        h = norm(x)
    ref = qlinear_grouped(h.contiguous(), qts, [None] * len(Ns), codes)
    out = qlinear_decode(x, qts, [None] * len(Ns), codes, mode, norm_weight=nw, norm_bias=nb, eps=eps)
    for o, b in zip(out, ref):
        _close(o, b, "norm prologue")
    again = qlinear_decode(x, qts, [None] * len(Ns), codes, mode, norm_weight=nw, norm_bias=nb, eps=eps)
    for o, b in zip(again, out):
        assert torch.equal(o, b)  # deterministic


def test_swiglu_prologue_crowded_tile_rows():
    """5 % outliers: a 16-row tile row holds thousands of entries: still bit
    for bit the separate launches' result."""
    M, N, K = 1, 256, 16384
    g = torch.Generator(device=DEV).manual_seed(9)
    w = torch.randn(N, K, generator=g, device=DEV) * 0.02
    m = torch.rand(N, K, generator=g, device=DEV) < 0.05
    w = torch.where(m, torch.sign(torch.randn(N, K, generator=g, device=DEV)) * 0.3, w).half()
    q = quantize_tensor(w, block_size=-1, code_format="e4m3")
    assert int(q.outlier_row_ptr[16].item()) > 2000  # the first tile row's entries
    codes = [kernel_codes(q, DEV)]
    gate = (torch.randn(M, K, generator=g, device=DEV) * 3).half()
    up = torch.randn(M, K, generator=g, device=DEV).half()
    a = torch.empty_like(gate)
    _lib.check(_lib.load().aq_silu_mul(gate.data_ptr(), up.data_ptr(), a.data_ptr(), M * K, _lib.stream_of(DEV)),
               "aq_silu_mul")
    ref = qlinear_grouped(a, [q], [None], codes)[0]
    assert torch.equal(qlinear_decode(a, [q], [None], codes)[0], ref)
    out = qlinear_decode(gate, [q], [None], codes, PRO_SWIGLU, x2=up)[0]
    assert torch.equal(out, ref)


def test_decode_entry_checks():
    """M = 1 (K within the x-in-LDS limit) or 6..64 rows, prologues on one
    row only, known prologues, the pieces each prologue needs, the
    residual not the output: refused before any launch."""
    qts = _weights([256], 1024, 7)
    codes = [kernel_codes(q, DEV) for q in qts]
    x = torch.randn(1, 1024, device=DEV).half()
    with pytest.raises(_lib.AQError, match="SwiGLU"):
        qlinear_decode(x, qts, [None], codes, PRO_SWIGLU)
    with pytest.raises(_lib.AQError, match="norm needs"):
        qlinear_decode(x, qts, [None], codes, PRO_RMS)
    with pytest.raises(_lib.AQError, match="LayerNorm needs"):
        qlinear_decode(x, qts, [None], codes, PRO_LAYERNORM, norm_weight=torch.ones(1024, device=DEV).half())
    with pytest.raises(_lib.AQError, match="unknown prologue"):
        qlinear_decode(x, qts, [None], codes, 9)
    x8 = torch.randn(8, 1024, device=DEV).half()
    with pytest.raises(_lib.AQError, match="prologues take one row"):
        qlinear_decode(x8, qts, [None], codes, PRO_RMS, norm_weight=torch.ones(1024, device=DEV).half())
    with pytest.raises(_lib.AQError, match="prologues take one row"):
        qlinear_decode(x8, qts, [None], codes, PRO_SWIGLU, x2=x8)
    with pytest.raises(_lib.AQError, match="6 <= M <= 64"):
        qlinear_decode(x8[:3].contiguous(), qts, [None], codes)
    pq = _weights([256, 256], 1024, 8)
    pc = [kernel_codes(q, DEV) for q in pq]
    with pytest.raises(_lib.AQError, match="SwiGLU pair"):
        qlinear_decode(x, pq, [None, None], pc, swiglu_pair=True)  # M = 1
    with pytest.raises(_lib.AQError, match="SwiGLU pair"):
        qlinear_decode(x8, pq, [None, None], pc, residuals=[x8[:, :256].contiguous(), None], swiglu_pair=True)
    with pytest.raises(ValueError, match="SwiGLU pair"):
        qlinear_decode(x8, qts, [None], codes, swiglu_pair=True)
    L = _lib.load()
    arr = _lib.ptr_array
    q = qts[0]
    y = torch.empty(1, 256, dtype=torch.float16, device=DEV)
    args = lambda res: (x.data_ptr(), 1, 1024, 1, 1, arr([256], ctypes.c_int64), arr([codes[0].data_ptr()]),  # noqa: E731
                        arr([q.scale_factors.data_ptr()]), arr([q.block_size], ctypes.c_int64),
                        arr([q.outlier_row_ptr.data_ptr()]), arr([_lib.ptr(q.outlier_cols)]),
                        arr([_lib.ptr(q.fp16_outliers)]), None, None, arr([None]), arr([y.data_ptr()]), PRO_NONE,
                        None, None, None,
                        ctypes.c_float(0.0), res, None, _lib.stream_of(DEV))
    with pytest.raises(_lib.AQError, match="must not be the output"):
        _lib.check(L.aq_qlinear_decode(*args(arr([y.data_ptr()]))), "aq_qlinear_decode")
