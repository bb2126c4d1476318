"""Live K/V summaries for residual tree nodes, on gfx950 (sparse/summaries.py:13-142).

``build_kv_summary_table(key, value, layout, *, block_size, prototypes,
token_mask=None)`` returns the reference's ``KVSummaryTable``: per tree node
``P`` positional prototypes, each the float32 mean of the valid key (value)
rows of one ``1/P`` slice of the node's token range, with the valid-token
counts and their logs (-inf for an empty slice).  The sums run in one HIP
pass over K and V (``spruce_kv_summary``), which builds a dyadic table of
16-token leaf sums and their pairwise sums; each range then adds the table
entries that cover it plus its partial leaves, one entry for a tree-node
prototype range, so upper tree levels do not re-read K/V.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

import spruce_hip
from interfaces.residual_summaries import ResidualTreeLayout
from sparse.config import SUMMARY_PROTOTYPES


@dataclass(frozen=True)
class KVSummaryTable:
    """Keys and values ``[B, Hkv, node, P, D]``; counts and log counts ``[B, node, P]``."""

    keys: torch.Tensor
    values: torch.Tensor
    counts: torch.Tensor
    log_counts: torch.Tensor
    range_starts: torch.Tensor
    range_ends: torch.Tensor


_RANGE_CACHE = {}


def _prototype_token_ranges(layout: ResidualTreeLayout, *, seq_len: int, block_size: int,
                            prototypes: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """Token ranges ``[node, P]``: slice p of node [s, e) is
    ``[s + len * p // P, s + len * (p + 1) // P)`` with the node's token range
    ``[start * block_size, end * block_size)`` clipped to ``seq_len``.  The
    tables depend only on the layout and sizes, so they are built once per
    device and reused (the layout is immutable)."""
    key = (layout.num_leaves, seq_len, block_size, prototypes, str(device))
    hit = _RANGE_CACHE.get(key)
    if hit is not None and hit[0] is layout:
        return hit[1], hit[2]
    starts, ends = _build_token_ranges(layout, seq_len, block_size, prototypes, device)
    _RANGE_CACHE[key] = (layout, starts, ends)
    return starts, ends


def _build_token_ranges(layout, seq_len, block_size, prototypes, device):
    first = (torch.tensor(layout.starts, device=device, dtype=torch.long) * block_size).clamp_max(seq_len)
    last = (torch.tensor(layout.ends, device=device, dtype=torch.long) * block_size).clamp_max(seq_len)
    length = (last - first)[:, None]
    p = torch.arange(prototypes, device=device, dtype=torch.long)[None, :]
    return first[:, None] + length * p // prototypes, first[:, None] + length * (p + 1) // prototypes


@torch.no_grad()
def build_kv_summary_table(key: torch.Tensor, value: torch.Tensor, layout: ResidualTreeLayout, *,
                           block_size: int, prototypes: int,
                           token_mask: torch.Tensor | None = None) -> KVSummaryTable:
    if key.dim() != 4 or value.dim() != 4:
        raise ValueError("key and value must be [batch, kv_heads, tokens, head_dim]")
    if key.shape != value.shape:
        raise ValueError(f"key/value shape mismatch: {key.shape} vs {value.shape}")
    if block_size < 1:
        raise ValueError(f"block_size must be positive, got {block_size}")
    if prototypes not in SUMMARY_PROTOTYPES:
        raise ValueError(f"prototypes must be one of {SUMMARY_PROTOTYPES}, got {prototypes}")
    batch, kv_heads, seq_len, head_dim = key.shape
    expected_leaves = (seq_len + block_size - 1) // block_size
    if layout.num_leaves != expected_leaves:
        raise ValueError(
            f"tree has {layout.num_leaves} leaves, expected {expected_leaves} "
            f"for seq_len={seq_len}, block_size={block_size}")
    valid = None
    if token_mask is not None:
        if token_mask.shape != (batch, seq_len):
            raise ValueError(f"token_mask must be {(batch, seq_len)}, got {tuple(token_mask.shape)}")
        valid = token_mask.to(device=key.device, dtype=torch.bool).contiguous().view(torch.uint8)
    if not key.is_cuda or not value.is_cuda:
        raise RuntimeError("build_kv_summary_table (HIP) requires GPU tensors")
    if value.dtype != key.dtype:
        raise ValueError("key and value must share a dtype")
    starts, ends = _prototype_token_ranges(layout, seq_len=seq_len, block_size=block_size,
                                           prototypes=prototypes, device=key.device)
    nodes = layout.num_nodes
    R = nodes * prototypes
    dev = key.device
    keys = torch.empty((batch, kv_heads, nodes, prototypes, head_dim), device=dev, dtype=torch.float32)
    values = torch.empty_like(keys)
    counts = torch.empty((batch, nodes, prototypes), device=dev, dtype=torch.float32)
    log_counts = torch.empty_like(counts)
    nbytes = spruce_hip.lib().spruce_kv_summary_workspace_bytes(batch, kv_heads, seq_len, head_dim)
    ws = torch.empty(max(nbytes, 1), device=dev, dtype=torch.uint8)
    s_flat, e_flat = starts.contiguous().view(-1), ends.contiguous().view(-1)
    with torch.cuda.device(dev):
        rc = spruce_hip.lib().spruce_kv_summary(
            spruce_hip.ptr(key), spruce_hip.strides(key), spruce_hip.ptr(value), spruce_hip.strides(value),
            batch, kv_heads, seq_len, head_dim, spruce_hip.dtype_code(key), spruce_hip.ptr(valid),
            spruce_hip.ptr(s_flat), spruce_hip.ptr(e_flat), R,
            spruce_hip.ptr(keys), spruce_hip.ptr(values), spruce_hip.ptr(counts), spruce_hip.ptr(log_counts),
            spruce_hip.ptr(ws), nbytes, spruce_hip.stream_of(key))
    spruce_hip.check(rc, "spruce_kv_summary")
    return KVSummaryTable(keys=keys, values=values, counts=counts, log_counts=log_counts,
                          range_starts=starts, range_ends=ends)


def token_validity_from_attention_mask(attention_mask: torch.Tensor | None, *, batch: int,
                                       seq_len: int) -> torch.Tensor | None:
    """Key padding validity ``[batch, seq_len]`` from a 4-D additive decoder mask:
    a key is real when at least one query row may attend to it."""
    if attention_mask is None:
        return None
    if attention_mask.dim() != 4:
        raise ValueError(
            "residual summaries expect a 4D additive attention mask, "
            f"got {tuple(attention_mask.shape)}")
    if attention_mask.shape[0] != batch or attention_mask.shape[-1] != seq_len:
        raise ValueError("attention mask batch/key dimensions do not match K/V")
    return (attention_mask[:, 0] >= 0).any(dim=-2)


def residual_attention_density(selected_blocks: torch.Tensor, residual_summary_nodes: torch.Tensor, *,
                               seq_len: int, block_size: int, prototypes: int) -> dict:
    """Attention entries a route charges (sparse/summaries.py:166-226):
    block_size per listed exact block plus one entry per listed node prototype
    whose token slice is non-empty, against the dense causal maximum."""
    if selected_blocks.dim() != 5 or residual_summary_nodes.dim() != 5:
        raise ValueError("selected and residual routes must both be 5D")
    if selected_blocks.shape[:4] != residual_summary_nodes.shape[:4]:
        raise ValueError("selected and residual routes must match through Q")
    if prototypes not in SUMMARY_PROTOTYPES:
        raise ValueError(f"prototypes must be one of {SUMMARY_PROTOTYPES}, got {prototypes}")
    batch, layers, groups, query_blocks, _ = selected_blocks.shape
    if query_blocks != (seq_len + block_size - 1) // block_size:
        raise ValueError("sequence length and route query-block count disagree")
    from interfaces.residual_summaries import build_residual_tree_layout

    tree = build_residual_tree_layout(query_blocks)
    first = (torch.tensor(tree.starts, dtype=torch.long) * block_size).clamp_max(seq_len)
    last = (torch.tensor(tree.ends, dtype=torch.long) * block_size).clamp_max(seq_len)
    # A node of n tokens split into P slices has min(P, n) non-empty ones.
    per_node = (last - first).clamp_max(prototypes)
    exact = int((selected_blocks >= 0).sum().item()) * block_size
    ids = residual_summary_nodes.detach().to(device="cpu", dtype=torch.long)
    ids = ids[ids >= 0]
    summary = int(per_node[ids].sum().item()) if ids.numel() else 0
    charged = exact + summary
    maximum = batch * layers * groups * query_blocks * (query_blocks + 1) // 2 * block_size
    fraction = charged / maximum if maximum else 0.0
    return {
        "exact_attention_entries": exact,
        "summary_prototype_entries": summary,
        "charged_attention_entries": charged,
        "maximum_causal_attention_entries": maximum,
        "charged_attention_fraction": fraction,
        "charged_sparsity": 1.0 - fraction,
    }
