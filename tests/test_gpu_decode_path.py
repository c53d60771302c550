"""QuantizedLinear's decode fast path (arguments prepared once per device,
weight and bias) gives the same bits as the stateless qlinear call, lies
within the north-star bounds of F.linear on the oracle's weight, and follows
a new bias, a new weight, a device move and every shape of x; inputs that
need gradients take the reference's F.linear path, whose backward reaches
x and the bias."""
import numpy as np
import pytest
import torch

import gpu_ref as R
from atlasinfer_core.quant import adaptive_quantizer as AQ
from integration import atlas_wrappers as AW

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _w(seed, N, K):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).half()
    w.view(-1)[torch.randperm(N * K, generator=g)[: N * K // 500]] *= 40
    return w


def _q(seed, N, K, fmt="e4m3", G=-1):
    return AQ.quantize_tensor(_w(seed, N, K).to(DEV), block_size=G, code_format=fmt)


def test_fast_path_matches_and_tracks_changes():
    N, K = 256, 1024
    q1, q2 = _q(1, N, K), _q(2, N, K, "int8", 128)
    b1 = torch.randn(N, device=DEV).half()
    b2 = torch.randn(N, device=DEV).half()
    ql = AW.QuantizedLinear(q1, b1)
    x = torch.randn(3, K, device=DEV).half()
    first = ql(x)                  # prepares the arguments
    assert ql._prep is not None
    w_ref = R.oracle_reference(q1, _w(1, N, K).numpy(), K, "e4m3")
    R.assert_close(first, R.reference_linear(x, w_ref, b1), x, w_ref)
    for _ in range(2):             # fast path
        assert torch.equal(ql(x), first)
    assert torch.equal(first, AW.qlinear(x, q1, b1))
    ql.bias = b2
    assert torch.equal(ql(x), AW.qlinear(x, q1, b2))
    ql.bias = None
    assert torch.equal(ql(x), AW.qlinear(x, q1, None))
    ql.quantized_weights = q2      # a new weight: codes and arguments rebuilt
    assert torch.equal(ql(x), AW.qlinear(x, q2, None))
    assert torch.equal(ql(x), AW.qlinear(x, q2, None))
    # shapes: 1-D, 3-D, a non-contiguous view, M past the GEMV, empty
    for xx in [x[0], x.view(1, 3, K), torch.randn(K, 4, device=DEV).half().t(),
               torch.randn(100, K, device=DEV).half(), torch.empty(0, K, device=DEV).half()]:
        assert torch.equal(ql(xx), AW.qlinear(xx, q2, None))
    with pytest.raises(RuntimeError):
        ql(x.float())
    with pytest.raises(RuntimeError):
        ql(torch.randn(2, K + 128, device=DEV).half())


def test_fast_path_after_module_move():
    q = _q(3, 128, 512)
    b = torch.randn(128).half()
    ql = AW.QuantizedLinear(q.to("cpu"), b).to(DEV)
    x = torch.randn(2, 512, device=DEV).half()
    y = ql(x)
    assert torch.equal(ql(x), y)
    assert torch.equal(y, AW.qlinear(x, q, b.to(DEV)))
    ql.to("cpu")
    with pytest.raises(RuntimeError):
        ql(x.cpu())
    ql.to(DEV)
    assert torch.equal(ql(x), y)


def test_inputs_needing_gradients_take_the_reference_path():
    """x.requires_grad (or a bias that does) under grad mode: y and the
    gradients are those of F.linear on the dequantized weight, as in the
    reference (atlas_wrappers.py:67); under no_grad the fused kernel runs."""
    N, K = 256, 1024
    q = _q(5, N, K)
    w_ref = R.oracle_reference(q, _w(5, N, K).numpy(), K, "e4m3")
    b = torch.randn(N, device=DEV).half()
    ql = AW.QuantizedLinear(q, b)
    x = torch.randn(4, K, device=DEV).half().requires_grad_()
    y = ql(x)
    assert y.requires_grad and y.grad_fn is not None
    dy = torch.randn_like(y)
    y.backward(dy)
    assert x.grad is not None
    gx = (dy.double() @ w_ref.double()).to(torch.float16)
    assert torch.allclose(x.grad.double(), gx.double(), rtol=2e-3, atol=2e-3)
    R.assert_close(y.detach(), R.reference_linear(x.detach(), w_ref, b), x.detach(), w_ref)
    bg = b.clone().requires_grad_()
    ql.bias = bg
    ql(x.detach()).sum().backward()
    assert bg.grad is not None and torch.all(bg.grad == 4)
    with torch.no_grad():
        assert not ql(x).requires_grad


def test_block_lists_built_only_for_calls_that_use_them():
    """A weight without stored block lists (int8, flat layout) gets them
    only when a call has LISTS_MIN_M rows or more: calls with fewer rows
    (decode at batch 1) build nothing, and so make no host sync; the
    arguments prepared before the lists existed are replaced once they do,
    and every call keeps the stateless call's bits.  The same holds for a
    sibling group's launch."""
    N, K = 256, 1024
    q = _q(7, N, K, "int8", 128)
    assert q.outlier_tile_ptr is None
    ql = AW.QuantizedLinear(q, None)
    x1 = torch.randn(1, K, device=DEV).half()
    x8 = torch.randn(8, K, device=DEV).half()
    for _ in range(3):
        assert torch.equal(ql(x1), AW.qlinear(x1, q, None))
    assert ql._tiles is None and ql._prep is not None and ql._prep[8] is None
    y8 = ql(x8)
    assert ql._tiles is not None and ql._prep[8] is not None
    assert torch.equal(y8, AW.qlinear(x8, q, None))
    assert torch.equal(ql(x8), y8)  # fast path with the lists
    assert torch.equal(ql(x1), AW.qlinear(x1, q, None))

    qa, qb = _q(8, N, K, "int8", 128), _q(9, N, K, "int8", 128)
    la, lb = AW.QuantizedLinear(qa, None), AW.QuantizedLinear(qb, None)
    g = AW.SiblingGroup([la, lb])
    la._group = lb._group = g
    ya = la(x1)
    assert la._tiles is None and lb._tiles is None
    assert torch.equal(ya, AW.qlinear(x1, qa, None)) and torch.equal(lb(x1), AW.qlinear(x1, qb, None))
    ya8 = la(x8)
    assert la._tiles is not None and lb._tiles is not None
    assert torch.equal(ya8, AW.qlinear(x8, qa, None)) and torch.equal(lb(x8), AW.qlinear(x8, qb, None))
