"""Import alias of atlasinfer_amd.quant under the reference's package path."""
