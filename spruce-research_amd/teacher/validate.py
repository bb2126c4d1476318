"""Causality check of a pooled level (teacher/validate.py:3-15)."""
import torch


def check_causal(pooled_layer, tolerance=1e-6):
    """(True, None) when no query block i puts more than ``tolerance`` of mass on a
    key block j > i; otherwise (False, (i, j)) for the first such cell in row-major
    order.  One reduction over batch and heads instead of a per-cell loop."""
    qb, kb = pooled_layer.shape[-2:]
    leak = pooled_layer.abs().amax(dim=tuple(range(pooled_layer.dim() - 2))) > tolerance
    leak &= torch.ones((qb, kb), dtype=torch.bool, device=leak.device).triu(diagonal=1)
    hits = leak.flatten().nonzero()
    if hits.numel() == 0:
        return True, None
    first = int(hits[0, 0])
    return False, (first // kb, first % kb)
