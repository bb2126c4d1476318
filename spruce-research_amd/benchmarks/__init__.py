"""Correctness gates of the sparse-prefill path (the reference's benchmarks/ package)."""
from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)
