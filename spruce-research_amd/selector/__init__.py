"""Selector front end (HIP): block pooling, gate scoring and causal top-k."""
