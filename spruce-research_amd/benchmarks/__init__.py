"""Correctness gates of the sparse-prefill path (the reference's benchmarks/ package)."""
