"""Import alias of atlasinfer_amd.integration under the reference's package name."""
