"""Import alias: the reference's package name for the quantization core.
The implementation is atlasinfer_amd.quant."""
