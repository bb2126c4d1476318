"""Sparse prefill attention (HIP-backed drop-in for the reference's sparse package)."""
