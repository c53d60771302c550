"""Import alias of atlasinfer_amd.utils under the reference's package path."""
