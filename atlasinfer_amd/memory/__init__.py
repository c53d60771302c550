"""Tiered key/value cache (HBM, page-locked host memory, disk)."""
