"""Import alias of atlasinfer_amd.memory under the reference's package path."""
