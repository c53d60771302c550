"""The reference's CPU path, restated op for op (TEST / BASELINE INFRASTRUCTURE).

Used only by bench.py's ``cpu_baseline`` leg (and tests).  It repeats the
reference's per-block torch loop and its forward so that their cost can be
timed on the GPU box's host cores; the reference itself never leaves the
build container.

* ``quantize_loop``    -- adaptive_quantizer.py:84-148 (one Python iteration
  per block, ~20 torch ops each)
* ``dequantize_loop``  -- adaptive_quantizer.py:175-245 (one Python iteration
  per block, each with a mask over ALL outlier indices and a host sync)
* ``forward_warm``     -- atlas_wrappers.py:67, F.linear on the cached fp16
  weight (the reference's steady state after the first call, :161-171)
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _zscore(data: torch.Tensor, eps=1e-6) -> torch.Tensor:  # :44-49
    mean = torch.mean(data)
    std = torch.std(data)
    return (data - mean) / (std + eps)


def quantize_loop(fp16_tensor: torch.Tensor, block_size: int = 128, z_threshold: float = 3.0,
                  max_blocks: int | None = None):
    """Per-block loop of quantize_tensor on CPU; stops after ``max_blocks``
    blocks (for time-boxed baselines).  Returns (codes, outliers, indices,
    scales, blocks_done)."""
    flat = fp16_tensor.flatten()
    n = flat.numel()
    padded = (n + block_size - 1) // block_size * block_size
    if padded > n:
        flat = torch.cat([flat, torch.zeros(padded - n, dtype=torch.float16)])
    blocks = flat.view(-1, block_size)
    nb = blocks.shape[0] if max_blocks is None else min(max_blocks, blocks.shape[0])
    codes, outs, idxs, scales = [], [], [], []
    for i in range(nb):
        block = blocks[i]
        z = _zscore(block)
        is_out = torch.abs(z) > z_threshold
        outs.append(block[is_out].clone())
        non = block[~is_out].clone()
        idxs.append(i * block_size + torch.where(is_out)[0])
        if non.numel() > 0:
            s = (torch.max(torch.abs(non)) / 127.0).clamp_(min=1e-6).to(torch.float16)
            q = torch.clamp(torch.round(non / s), min=-127.0, max=127.0).to(torch.int8)
        else:
            q = torch.empty((0,), dtype=torch.int8)
            s = torch.tensor(1.0, dtype=torch.float16)
        codes.append(q)
        scales.append(s.unsqueeze(0))
    return torch.cat(codes), torch.cat(outs), torch.cat(idxs), torch.cat(scales), nb


def dequantize_loop(fp8_data: torch.Tensor, fp16_outliers: torch.Tensor, outlier_indices: torch.Tensor,
                    scale_factors: torch.Tensor, numel: int, block_size: int, max_blocks: int | None = None,
                    progress=None, every: int = 16384):
    """Per-block loop of dequantize_tensor on CPU (the reference's int8
    layout: compacted codes of the non-outliers); stops after ``max_blocks``
    blocks.  ``progress(blocks_done, blocks)`` is called every ``every``
    blocks (long runs report as they go).  Returns (flat fp16 tensor of the
    padded length, blocks_done)."""
    padded = (numel + block_size - 1) // block_size * block_size
    nb = padded // block_size if max_blocks is None else min(max_blocks, padded // block_size)
    out = torch.zeros(padded, dtype=torch.float16)
    pos = 0
    for i in range(nb):
        s = scale_factors[i]
        b0, b1 = i * block_size, (i + 1) * block_size
        in_block = (outlier_indices >= b0) & (outlier_indices < b1)  # :194-196, over all outliers
        sel = torch.where(in_block)[0]
        rel = outlier_indices[in_block] - b0
        vals = fp16_outliers[sel]
        n_codes = max(block_size - rel.numel(), 0)
        codes = fp8_data[pos:pos + n_codes]
        pos += n_codes
        deq = codes.to(torch.float16) * s if n_codes > 0 else torch.empty((0,), dtype=torch.float16)
        blk = torch.zeros(block_size, dtype=torch.float16)
        keep = torch.ones(block_size, dtype=torch.bool)
        if rel.numel() > 0:
            keep[rel] = False
            blk[rel] = vals
        n_keep = keep.sum().item()  # :234, the host sync of every block
        blk[keep] = deq[:n_keep]
        out[b0:b1] = blk
        if progress is not None and (i + 1) % every == 0:
            progress(i + 1, nb)
    return out, nb


def forward_warm(x: torch.Tensor, w_fp16: torch.Tensor, bias=None) -> torch.Tensor:
    return F.linear(x, w_fp16, bias)
