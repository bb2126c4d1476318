"""Leaf-first binary key tree and residual frontiers (interfaces/residual_summaries.py:19-313).

Node IDs are stable and leaf-first: level 0 holds one node per key block,
each higher level ``ceil(previous / 2)`` nodes, and node ``(level, i)`` has ID
``level_offsets[level] + i``.  Its leaf range is
``[i * 2**level, min((i + 1) * 2**level, num_leaves))`` -- the union of its
children ``2i`` and ``2i + 1`` (an odd tail node has one child).  The field
names and ID order are the reference's, so node IDs exchanged with it agree.

A row's residual frontier is the set of maximal nodes covering the causal
blocks [0, q] its selected_blocks row does not list.  Calling a node
"blocked" when its range holds a listed block or reaches past q, the frontier
is every unblocked node whose parent is blocked (or that is the root):
blocked propagates to parents, so this is the set the reference's top-down
visit collects.  ``build_residual_summary_nodes`` computes it for all rows in
one HIP launch (``spruce_residual_frontier``); ``residual_frontier_for_row``
is the single-row host form; ``validate_residual_summary_nodes`` checks every
rule of the reference's validator for every row with tensor ops and reports
the first violation in row order with the reference's message.
"""
from __future__ import annotations

import functools
from dataclasses import dataclass
from typing import Iterable, Sequence

import torch

import spruce_hip
from interfaces.validator import PAD_VALUE, validate_selected_blocks


@dataclass(frozen=True)
class ResidualTreeLayout:
    num_leaves: int
    level_counts: tuple[int, ...]
    level_offsets: tuple[int, ...]
    starts: tuple[int, ...]
    ends: tuple[int, ...]
    levels: tuple[int, ...]
    indices: tuple[int, ...]

    @property
    def num_nodes(self) -> int:
        return len(self.starts)

    @property
    def root_id(self) -> int:
        return self.level_offsets[-1]

    def node_id(self, level: int, index: int) -> int:
        if not 0 <= level < len(self.level_counts):
            raise IndexError(f"tree level {level} is out of range")
        if not 0 <= index < self.level_counts[level]:
            raise IndexError(f"node index {index} is out of range for level {level}")
        return self.level_offsets[level] + index

    def range(self, node_id: int) -> tuple[int, int]:
        if not 0 <= node_id < self.num_nodes:
            raise IndexError(f"tree node ID {node_id} is out of range")
        return self.starts[node_id], self.ends[node_id]

    def children(self, node_id: int) -> tuple[int, ...]:
        if not 0 <= node_id < self.num_nodes:
            raise IndexError(f"tree node ID {node_id} is out of range")
        level = self.levels[node_id]
        if level == 0:
            return ()
        below = level - 1
        first = 2 * self.indices[node_id]
        return tuple(self.level_offsets[below] + c for c in (first, first + 1)
                     if c < self.level_counts[below])


def build_residual_tree_layout(num_leaves: int) -> ResidualTreeLayout:
    """Node ID and leaf-range table of the tree over ``num_leaves`` key blocks.

    The layout depends only on the leaf count and is immutable, so each count
    is built once (a layer's attention call asks for it every time)."""
    if num_leaves < 1:
        raise ValueError(f"num_leaves must be >= 1, got {num_leaves}")
    return _tree_layout(int(num_leaves))


@functools.lru_cache(maxsize=64)
def _tree_layout(n: int) -> ResidualTreeLayout:
    counts = [n]
    while counts[-1] > 1:
        counts.append((counts[-1] + 1) // 2)
    offsets = [sum(counts[:lvl]) for lvl in range(len(counts))]
    starts, ends, levels, indices = [], [], [], []
    for level, count in enumerate(counts):
        width = 1 << level
        for i in range(count):
            starts.append(i * width)
            ends.append(min((i + 1) * width, n))
            levels.append(level)
            indices.append(i)
    return ResidualTreeLayout(n, tuple(counts), tuple(offsets), tuple(starts), tuple(ends),
                              tuple(levels), tuple(indices))


def residual_frontier_for_row(selected_block_ids: Sequence[int] | Iterable[int], query_block: int,
                              layout: ResidualTreeLayout) -> list[int]:
    """Maximal nodes covering the causal blocks of row ``query_block`` that
    ``selected_block_ids`` omits, ascending by node ID (negative IDs ignored)."""
    if not 0 <= query_block < layout.num_leaves:
        raise ValueError(f"query_block must be in [0, {layout.num_leaves}), got {query_block}")
    listed = sorted({int(b) for b in selected_block_ids if b >= 0})
    if listed and listed[-1] > query_block:
        raise ValueError("selected block IDs must be causal and non-negative")
    end_causal = query_block + 1
    # prefix[j] = listed blocks below j, so a range [s, e) holds one iff prefix differs.
    prefix = [0] * (end_causal + 1)
    for j in listed:
        prefix[j + 1] += 1
    for j in range(end_causal):
        prefix[j + 1] += prefix[j]

    def blocked(node: int) -> bool:
        s, e = layout.starts[node], layout.ends[node]
        return e > end_causal or prefix[e] > prefix[s]

    top = len(layout.level_counts) - 1
    frontier = []
    for level, (count, offset) in enumerate(zip(layout.level_counts, layout.level_offsets)):
        for i in range(count):
            node = offset + i
            if layout.starts[node] >= end_causal:
                break
            if blocked(node):
                continue
            if level == top or blocked(layout.level_offsets[level + 1] + i // 2):
                frontier.append(node)
    return frontier


def _frontier_device(selected_blocks: torch.Tensor) -> torch.device:
    if selected_blocks.is_cuda:
        return selected_blocks.device
    if torch.cuda.is_available():
        return torch.device("cuda", torch.cuda.current_device())
    raise RuntimeError("build_residual_summary_nodes runs on the GPU (spruce_residual_frontier); "
                       "no GPU is available")


@torch.no_grad()
def build_residual_summary_nodes(selected_blocks: torch.Tensor, *,
                                 layout: ResidualTreeLayout | None = None,
                                 validate_selected: bool = True) -> torch.Tensor:
    """``[B,L,G,Q,S]`` int32 residual frontiers, ``S`` = the largest frontier,
    trailing ``-1`` padding (``S == 0`` when every row lists all its blocks).
    Returned on ``selected_blocks``' device."""
    if validate_selected:
        validate_selected_blocks(selected_blocks)
    if selected_blocks.dim() != 5:
        raise ValueError("selected_blocks must be [B,L,G,Q,K]")
    if selected_blocks.dtype != torch.int32:
        raise ValueError(f"selected_blocks must be int32, got {selected_blocks.dtype}")
    batch, layers, groups, query_blocks, width = selected_blocks.shape
    if layout is None:
        layout = build_residual_tree_layout(query_blocks) if query_blocks else None
    elif layout.num_leaves != query_blocks:
        raise ValueError(
            f"tree has {layout.num_leaves} leaves but selected_blocks has "
            f"{query_blocks} query blocks")
    rows = batch * layers * groups * query_blocks
    if rows == 0:
        return torch.full((batch, layers, groups, query_blocks, 0), PAD_VALUE, dtype=torch.int32,
                          device=selected_blocks.device)
    dev = _frontier_device(selected_blocks)
    sel = selected_blocks.to(dev)
    counts = torch.empty(rows, dtype=torch.int32, device=dev)
    lib = spruce_hip.lib()
    with torch.cuda.device(dev):
        stream = spruce_hip.stream_of(sel)
        args = (spruce_hip.ptr(sel), spruce_hip.strides5(sel), batch, layers, groups, query_blocks, width)
        spruce_hip.check(lib.spruce_residual_frontier(*args, spruce_hip.ptr(counts), None, 0, stream),
                         "spruce_residual_frontier")
        if rows and int(counts.min()) < 0:
            raise ValueError("selected block IDs must be causal and non-negative")
        largest = int(counts.max()) if rows else 0
        out = torch.empty((batch, layers, groups, query_blocks, largest), dtype=torch.int32, device=dev)
        if largest:
            spruce_hip.check(lib.spruce_residual_frontier(*args, spruce_hip.ptr(counts), spruce_hip.ptr(out),
                                                          largest, stream), "spruce_residual_frontier")
    return out.to(selected_blocks.device)


def _location(row: int, groups: int, layers: int, query_blocks: int) -> str:
    q = row % query_blocks
    g = (row // query_blocks) % groups
    l = (row // (query_blocks * groups)) % layers
    b = row // (query_blocks * groups * layers)
    return f"b={b}, l={l}, g={g}, q={q}"


@torch.no_grad()
def validate_residual_summary_nodes(selected_blocks: torch.Tensor, residual_summary_nodes: torch.Tensor, *,
                                    require_maximal: bool = True, validate_selected: bool = True) -> None:
    """Raise AssertionError unless, in every row, the exact blocks and the
    residual nodes partition the causal prefix [0, q] (and, with
    ``require_maximal``, the nodes are the maximal frontier)."""
    if validate_selected:
        validate_selected_blocks(selected_blocks)
    assert residual_summary_nodes.dim() == 5, (
        "Expected residual_summary_nodes [batch, layer, kv_head_group, "
        f"query_block, S], got {tuple(residual_summary_nodes.shape)}")
    assert residual_summary_nodes.dtype == torch.int32, (
        f"Expected residual_summary_nodes int32, got {residual_summary_nodes.dtype}")
    assert residual_summary_nodes.shape[:4] == selected_blocks.shape[:4], (
        "selected_blocks and residual_summary_nodes must have identical "
        "[batch, layer, group, query] dimensions, got "
        f"{tuple(selected_blocks.shape[:4])} and {tuple(residual_summary_nodes.shape[:4])}")
    batch, layers, groups, query_blocks, _ = selected_blocks.shape
    rows = batch * layers * groups * query_blocks
    if rows == 0:
        return
    dev = selected_blocks.device
    layout = build_residual_tree_layout(query_blocks)
    nnodes = layout.num_nodes
    starts = torch.tensor(layout.starts, device=dev, dtype=torch.long)
    ends = torch.tensor(layout.ends, device=dev, dtype=torch.long)
    levels = torch.tensor(layout.levels, device=dev, dtype=torch.long)
    lvl_off = torch.tensor(layout.level_offsets, device=dev, dtype=torch.long)
    top = len(layout.level_counts) - 1

    exact = selected_blocks.reshape(rows, -1).to(torch.long)
    res = residual_summary_nodes.to(dev).reshape(rows, -1).to(torch.long)
    S = res.shape[1]
    qv = torch.arange(query_blocks, device=dev).repeat(rows // query_blocks)[:, None]

    # Rule codes in the reference's per-row order: 1 padding, 2 sorted,
    # 3 duplicates, 4 exact causal / node known / node causal, 5 partition,
    # 6 maximal.
    pad = res == PAD_VALUE
    real = ~pad
    bad_pad = (real & (pad.to(torch.int32).cumsum(dim=-1) > 0)).any(dim=-1)
    both = real[:, 1:] & real[:, :-1]
    unsorted = ((res[:, 1:] < res[:, :-1]) & both).any(dim=-1)
    dup = ((res[:, 1:] == res[:, :-1]) & both).any(dim=-1)
    ex_real = exact != PAD_VALUE
    bad_exact = (ex_real & ((exact < 0) | (exact > qv))).any(dim=-1)
    known = (res >= 0) & (res < nnodes)
    nid = res.clamp(0, max(nnodes - 1, 0))
    future = known & (ends[nid] > qv + 1)
    bad_node = (real & (~known | future)).any(dim=-1)

    # Coverage of [0, q] by exact blocks and node ranges: difference arrays,
    # in row chunks to bound memory.
    bad_cov = torch.zeros(rows, dtype=torch.bool, device=dev)
    bad_max = torch.zeros(rows, dtype=torch.bool, device=dev)
    width = query_blocks + 2
    chunk = max(1, (1 << 24) // width)
    col = torch.arange(query_blocks, device=dev)[None, :]
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        n = r1 - r0
        base = torch.arange(n, device=dev)[:, None] * width
        ex = exact[r0:r1]
        exv = ex_real[r0:r1] & (ex >= 0) & (ex <= qv[r0:r1])
        exi = ex.clamp(0, query_blocks - 1)
        ediff = torch.zeros(n * width, dtype=torch.int32, device=dev)
        ones = exv.to(torch.int32)
        ediff.scatter_add_(0, (base + exi).reshape(-1), ones.reshape(-1))
        ediff.scatter_add_(0, (base + exi + 1).reshape(-1), -ones.reshape(-1))
        nv = real[r0:r1] & known[r0:r1] & ~future[r0:r1]
        nn = nid[r0:r1]
        cdiff = ediff.clone()
        w = nv.to(torch.int32)
        cdiff.scatter_add_(0, (base + starts[nn]).reshape(-1), w.reshape(-1))
        cdiff.scatter_add_(0, (base + ends[nn]).reshape(-1), -w.reshape(-1))
        cov = cdiff.view(n, width).cumsum(dim=-1)[:, :query_blocks]
        bad_cov[r0:r1] = ((cov != 1) & (col <= qv[r0:r1])).any(dim=-1)
        if require_maximal:
            # A node is maximal iff its parent is blocked: the parent's range
            # reaches past q or holds an exact block (the root has no parent).
            eprefix = torch.cat([torch.zeros(n, 1, dtype=torch.int32, device=dev),
                                 ediff.view(n, width).cumsum(dim=-1).clamp_max(1).cumsum(dim=-1)], dim=-1)
            lv = levels[nn]
            is_root = lv >= top
            pidx = lvl_off[(lv + 1).clamp_max(top)] + (nn - lvl_off[lv]) // 2
            ps, pe = starts[pidx], ends[pidx]
            holds = eprefix.gather(1, pe) > eprefix.gather(1, ps)
            pblocked = is_root | (pe > qv[r0:r1] + 1) | holds
            bad_max[r0:r1] = (nv & ~pblocked).any(dim=-1)

    codes = torch.stack([bad_pad, unsorted, dup, bad_exact | bad_node, bad_cov, bad_max], dim=-1)
    failing = codes.any(dim=-1)
    if not bool(failing.any()):
        return
    row = int(torch.nonzero(failing)[0, 0])
    rule = int(torch.nonzero(codes[row])[0, 0])
    loc = _location(row, groups, layers, query_blocks)
    ex_row = [int(x) for x in exact[row].tolist() if x != PAD_VALUE]
    padded = [int(x) for x in res[row].tolist()]
    residual = [x for x in padded if x != PAD_VALUE]
    q = row % query_blocks
    if rule == 0:
        raise AssertionError(f"Residual padding is not trailing-only at [{loc}]")
    if rule == 1:
        raise AssertionError(f"Residual node IDs are not sorted at [{loc}]: {residual}")
    if rule == 2:
        raise AssertionError(f"Duplicate residual node IDs at [{loc}]: {residual}")
    if rule == 3:
        for block_id in ex_row:
            if not 0 <= block_id <= q:
                raise AssertionError(f"Non-causal exact block {block_id} at [{loc}]")
        for node_id in residual:
            if not 0 <= node_id < nnodes:
                raise AssertionError(f"Unknown residual node ID {node_id} at [{loc}]")
            start, end = layout.range(node_id)
            if end > q + 1:
                raise AssertionError(
                    f"Residual node {node_id} range [{start}, {end}) is partially or wholly "
                    f"future at [{loc}]")
    if rule == 4:
        coverage = [0] * (q + 1)
        for block_id in ex_row:
            coverage[block_id] += 1
        for node_id in residual:
            start, end = layout.range(node_id)
            for block_id in range(start, end):
                coverage[block_id] += 1
        raise AssertionError(
            "Exact and residual routes do not form a disjoint complete causal partition "
            f"at [{loc}]: coverage={coverage}")
    expected = residual_frontier_for_row(ex_row, q, layout)
    raise AssertionError(
        f"Residual frontier is complete but not maximal at [{loc}]: expected {expected}, "
        f"got {residual}")
