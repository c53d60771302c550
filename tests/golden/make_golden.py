"""Writes the golden fixtures in this directory from the reference itself.

Run in the build container (where the reference is mounted read-only at
/root/reference):  python tests/golden/make_golden.py

Why an import is needed: the reference's own tests
(/root/reference/tests/test_quantizer.py:40,49,56) only assert MSE < 1e-3 and
a shape, so nothing in the reference pins the bit-level output of
quantize_tensor / dequantize_tensor / calculate_zscore_manual.  This script
calls those three functions (adaptive_quantizer.py:44,51,156) on small seeded
inputs and stores inputs and outputs as .npz data; the reference never leaves
this container, only these vectors do.

Each case file holds: x (fp16 input), block_size, z_threshold, and the
reference's fp8_data (int8), fp16_outliers, outlier_indices (int64),
scale_factors (fp16), deq (dequantize_tensor output, fp16).  zscore.npz holds
calculate_zscore_manual inputs/outputs.
"""
import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference/atlasinfer_core/quant/adaptive_quantizer.py"


def load_reference():
    spec = importlib.util.spec_from_file_location("_reference_adaptive_quantizer", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def weights(gen, shape, sigma=0.02, outlier_frac=0.001, t_dof=None):
    """fp16 weights: N(0, sigma) (or Student-t * sigma) with a fraction of
    entries replaced by sign * U(8, 20) * sigma (the BASELINE distribution)."""
    n = int(np.prod(shape))
    if t_dof is None:
        w = torch.randn(n, generator=gen) * sigma
    else:
        z = torch.randn(n, generator=gen)
        chi = (torch.randn(n, t_dof, generator=gen) ** 2).sum(1) / t_dof
        w = z / chi.sqrt() * sigma
    k = int(round(outlier_frac * n))
    if k:
        pos = torch.randperm(n, generator=gen)[:k]
        sign = torch.where(torch.rand(k, generator=gen) < 0.5, -1.0, 1.0)
        mag = (torch.rand(k, generator=gen) * 12 + 8) * sigma
        w[pos] = sign * mag
    return w.reshape(shape).to(torch.float16)


def cases():
    g = torch.Generator().manual_seed(1234)
    out = []
    # 1. the reference test's own standard case (test_quantizer.py:13-22)
    t = (torch.randn(128, 256, generator=g) * 5).to(torch.float16)
    t.view(-1)[::150] *= 10
    out.append(("ref_test_standard", t, 64, 3.5))
    # 2. smaller than one block (test_quantizer.py:44-46)
    out.append(("ref_test_small", torch.randn(10, generator=g).to(torch.float16), 64, 3.0))
    # 3. OPT-like weights, reference default block 128
    out.append(("opt_like_g128", weights(g, (64, 256)), 128, 3.0))
    # 4. one block per row (per-output-channel), K = 512
    out.append(("per_row_k512", weights(g, (48, 512)), 512, 3.0))
    # 5. heavy tails (Student-t, 1% outliers)
    out.append(("student_t_g128", weights(g, (32, 256), outlier_frac=0.01, t_dof=3), 128, 3.0))
    # 6. block size not dividing the tensor, odd length
    out.append(("g100_ragged", weights(g, (1003,)), 100, 3.0))
    # 7. threshold that is not exact in fp16 (rounds to 3.30078125)
    out.append(("thr_3p3", weights(g, (16, 256)), 128, 3.3))
    # 8. large magnitudes, scale far from 1
    out.append(("large_values", (torch.randn(8, 256, generator=g) * 900).to(torch.float16), 128, 3.0))
    # 9. tiny magnitudes: subnormal fp16 inputs, scale clamped at fp16(1e-6)
    tiny = (torch.randn(4, 128, generator=g) * 2e-6).to(torch.float16)
    out.append(("tiny_values", tiny, 64, 3.0))
    # 10. edge blocks: constant, zeros, one spike, alternating signs
    e = torch.zeros(6, 64)
    e[0] = 0.5
    e[2, 17] = 3.0
    e[3] = torch.tensor([1.0, -1.0] * 32)
    e[4] = torch.linspace(-2, 2, 64)
    e[5, :] = 0.01
    e[5, ::9] = 7.0
    out.append(("edge_blocks", e.to(torch.float16), 64, 3.0))
    # 11. low threshold (many outliers per block)
    out.append(("low_threshold", weights(g, (16, 128)), 32, 1.0))
    # 12. block of 8, small groups
    out.append(("g8", weights(g, (8, 64), outlier_frac=0.02), 8, 2.0))
    # 13-14. bulk: many blocks, to exercise the fp16 mean/std rounding
    out.append(("bulk_g128", weights(g, (256, 512)), 128, 3.0))
    out.append(("bulk_per_row_k1024", weights(g, (128, 1024), outlier_frac=0.01, t_dof=3), 1024, 3.0))
    # 15-18. rows at the block sizes the product runs (one block per output
    # channel of the Llama-3-8B shapes: K = 4096 and 14336), normal and
    # Student-t weights; their own generator, so cases 1-14 stay as they were
    g2 = torch.Generator().manual_seed(4096)
    out.append(("per_row_k4096", weights(g2, (8, 4096)), 4096, 3.0))
    out.append(("per_row_k4096_t3", weights(g2, (8, 4096), outlier_frac=0.01, t_dof=3), 4096, 3.0))
    out.append(("per_row_k14336", weights(g2, (4, 14336)), 14336, 3.0))
    out.append(("per_row_k14336_t3", weights(g2, (2, 14336), outlier_frac=0.01, t_dof=3), 14336, 3.0))
    return out


def main():
    ref = load_reference()
    torch.manual_seed(0)
    for name, t, G, thr in cases():
        qt = ref.quantize_tensor(t.clone(), block_size=G, z_threshold=thr)
        # the reference memoises by id(QuantizedTensor); ids of collected
        # tuples are reused, so clear it or a stale tensor comes back
        ref.clear_dequantized_cache()
        deq = ref.dequantize_tensor(qt, torch.device("cpu"))
        assert tuple(deq.shape) == tuple(t.shape)
        np.savez_compressed(
            os.path.join(HERE, f"{name}.npz"),
            x=t.numpy(),
            block_size=np.int64(G),
            z_threshold=np.float64(thr),
            fp8_data=qt.fp8_data.numpy(),
            fp16_outliers=qt.fp16_outliers.numpy(),
            outlier_indices=qt.outlier_indices.numpy(),
            scale_factors=qt.scale_factors.numpy(),
            deq=deq.numpy(),
        )
        print(f"{name}: shape={tuple(t.shape)} G={G} thr={thr} nnz={qt.outlier_indices.numel()} "
              f"codes={qt.fp8_data.numel()}")
    # calculate_zscore_manual on a few 1-D fp16 tensors
    g = torch.Generator().manual_seed(99)
    zs_in, zs_out, lens = [], [], []
    for n, scale in [(128, 0.02), (64, 5.0), (4096, 0.02), (7, 1.0), (1000, 300.0)]:
        x = (torch.randn(n, generator=g) * scale).to(torch.float16)
        z = ref.calculate_zscore_manual(x)
        zs_in.append(x.numpy())
        zs_out.append(z.numpy())
        lens.append(n)
    np.savez(os.path.join(HERE, "zscore.npz"), lens=np.array(lens, np.int64),
             x=np.concatenate(zs_in), z=np.concatenate(zs_out))
    print("torch", torch.__version__)
    with open(os.path.join(HERE, "VERSIONS.txt"), "w") as f:
        f.write(f"torch {torch.__version__}\nnumpy {np.__version__}\npython {sys.version.split()[0]}\n")


if __name__ == "__main__":
    main()
