"""Key-axis prototype tree on gfx950 (selector/tree.py:17-145, 203-254).

``build_key_tree(k_feat [L,G,kb,P,d], radix=2)`` returns the levels
leaf-first as ``KeyTreeLevel`` (level, features, starts, ends), like the
reference.  All levels come from one library call
(``spruce_tree_merge_levels``: a launch per wide level, the narrow levels near
the root in one launch):
per parent, prototype 0 is the mean of its children's prototype 0 (summed and
divided in the model dtype, as the reference does) and prototypes 1..P-1 are
the child prototypes farthest from it, farthest first.  Node ranges: node i of
level v covers leaf blocks [i * radix**v, min((i + 1) * radix**v, kb)), the
reference's odd-tail rollup.

Differences, documented: distances are float32 (the reference computes them
in the model dtype) and equal distances go to the lower child prototype (the
reference leaves tie order to ``torch.topk``).

The target-side tree and the tree-KL training loss of the reference module
(``TargetTreeLevel``, ``build_target_tree``, ``iter_tree_levels``,
``tree_kl_loss``, selector/tree.py:32-43, 148-202, 219-291, 305-) are not part
of the inference path: those names come from the checkout's selector/tree.py
through the module ``__getattr__``.
"""
import ctypes
from dataclasses import dataclass

import torch

import spruce_hip
from spruce_hip.overlay import forward_missing

__getattr__ = forward_missing("selector.tree", __file__)


@dataclass(frozen=True)
class KeyTreeLevel:
    """Key-node features of one tree level.

    features: [L, G, num_nodes, P, d]; starts/ends: [num_nodes] leaf-block
    half-open intervals [start, end).
    """
    level: int
    features: torch.Tensor
    starts: torch.Tensor
    ends: torch.Tensor


def _validate_radix(radix):
    if radix < 2:
        raise ValueError(f"radix must be >= 2, got {radix}")


def tree_node_counts(num_leaf_nodes, radix=2, include_root=False):
    """Leaf-first node counts of the fixed key tree (selector/tree.py:203-215)."""
    _validate_radix(radix)
    if num_leaf_nodes < 1:
        raise ValueError("num_leaf_nodes must be >= 1")
    counts = []
    nodes = int(num_leaf_nodes)
    while nodes > 1:
        counts.append(nodes)
        nodes = (nodes + radix - 1) // radix
    if include_root:
        counts.append(1)
    return counts


def level_ranges(num_leaves, level, radix, device=None):
    """(starts, ends) int64 leaf ranges of every node of one level."""
    span = radix ** level
    count = num_leaves
    for _ in range(level):
        count = (count + radix - 1) // radix
    starts = torch.arange(count, device=device, dtype=torch.long) * span
    return starts, (starts + span).clamp_max(num_leaves)


_RANGE_TABLES = {}


def _level_range_table(num_leaves, radix, device):
    """level_ranges of every level (leaf first), computed on the host and
    moved to the device in one copy; returns per-level (starts, ends) views.

    The table depends only on (num_leaves, radix, device), so it is built once
    per key and shared by every tree built after (its host-to-device copy
    would otherwise stall the host behind the GPU on every call); the range
    tensors must not be modified in place."""
    key = (int(num_leaves), int(radix), str(torch.device(device)))
    hit = _RANGE_TABLES.get(key)
    if hit is None:
        hit = _RANGE_TABLES[key] = _build_level_range_table(num_leaves, radix, device)
    return hit


def _build_level_range_table(num_leaves, radix, device):
    counts, spans = [num_leaves], [1]
    while counts[-1] > 1:
        counts.append((counts[-1] + radix - 1) // radix)
        spans.append(spans[-1] * radix)
    starts = torch.cat([torch.arange(c, dtype=torch.long) * sp for c, sp in zip(counts, spans)])
    widths = torch.repeat_interleave(torch.tensor(spans, dtype=torch.long), torch.tensor(counts))
    table = torch.stack([starts, (starts + widths).clamp_max(num_leaves)]).to(device)
    out, off = [], 0
    for c in counts:
        out.append((table[0, off:off + c], table[1, off:off + c]))
        off += c
    return out


def merge_level(features, radix=2):
    """One parent level: [L,G,n,P,d] -> [L,G,ceil(n/radix),P,d] (HIP)."""
    _validate_radix(radix)
    if features.dim() != 5:
        raise ValueError(f"features must be [L,G,n,P,d], got {tuple(features.shape)}")
    if not features.is_cuda:
        raise RuntimeError("build_key_tree (HIP) requires GPU tensors")
    L, G, n, P, d = features.shape
    x = features.contiguous()
    out = torch.empty((L, G, (n + radix - 1) // radix, P, d), device=x.device, dtype=x.dtype)
    with torch.cuda.device(x.device):
        rc = spruce_hip.lib().spruce_tree_merge_level(
            spruce_hip.ptr(x), L * G, n, P, d, radix, spruce_hip.dtype_code(x), spruce_hip.ptr(out),
            spruce_hip.stream_of(x))
    spruce_hip.check(rc, "spruce_tree_merge_level")
    return out


def merge_levels(features, radix=2):
    """Every parent level above ``features`` up to the root, from one library
    call (``spruce_tree_merge_levels``: a launch per wide level, then the
    narrow levels near the root in one launch); each level equals what
    :func:`merge_level` gives for it."""
    _validate_radix(radix)
    if features.dim() != 5:
        raise ValueError(f"features must be [L,G,n,P,d], got {tuple(features.shape)}")
    if not features.is_cuda:
        raise RuntimeError("build_key_tree (HIP) requires GPU tensors")
    L, G, n, P, d = features.shape
    x = features.contiguous()
    outs = []
    while n > 1:
        n = (n + radix - 1) // radix
        outs.append(torch.empty((L, G, n, P, d), device=x.device, dtype=x.dtype))
    if not outs:
        return outs
    ptrs = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    with torch.cuda.device(x.device):
        rc = spruce_hip.lib().spruce_tree_merge_levels(
            spruce_hip.ptr(x), L * G, x.shape[2], P, d, radix, spruce_hip.dtype_code(x), ptrs, len(outs),
            spruce_hip.stream_of(x))
    spruce_hip.check(rc, "spruce_tree_merge_levels")
    return outs


@torch.no_grad()
def build_key_tree(k_feat, radix=2):
    """Key-node feature levels, leaf-first; odd tails become smaller parents."""
    _validate_radix(radix)
    if k_feat.dim() != 5:
        raise ValueError(f"k_feat must be [L,G,kb,P,d], got {tuple(k_feat.shape)}")
    kb = k_feat.shape[2]
    ranges = _level_range_table(kb, radix, k_feat.device)
    levels = [KeyTreeLevel(0, k_feat, *ranges[0])]
    for level, out in enumerate(merge_levels(k_feat, radix), start=1):
        levels.append(KeyTreeLevel(level, out, *ranges[level]))
    return levels


def ancestor_node_id(leaf_block, starts, ends):
    """The unique node whose half-open range contains ``leaf_block``, or -1."""
    leaf_block = int(leaf_block)
    if leaf_block < 0:
        return -1
    matches = (starts <= leaf_block) & (leaf_block < ends)
    indices = matches.nonzero(as_tuple=False).flatten()
    if indices.numel() != 1:
        return -1
    return int(indices.item())
