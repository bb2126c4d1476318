"""Selector front end (HIP): block pooling, gate scoring and causal top-k."""
from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)
