"""Quantization core (reference: atlasinfer_core/quant)."""
