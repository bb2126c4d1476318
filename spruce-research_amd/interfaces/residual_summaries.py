"""Leaf-first binary key tree for residual summaries (interfaces/residual_summaries.py:19-117).

Node IDs are stable and leaf-first: level 0 holds one node per key block,
each higher level ``ceil(previous / 2)`` nodes, and node ``(level, i)`` has ID
``level_offsets[level] + i``.  Its leaf range is
``[i * 2**level, min((i + 1) * 2**level, num_leaves))`` -- the union of its
children ``2i`` and ``2i + 1`` (an odd tail node has one child).  The field
names and ID order are the reference's, so node IDs exchanged with it agree.
"""
from __future__ import annotations

from dataclasses import dataclass


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
    """Node ID and leaf-range table of the tree over ``num_leaves`` key blocks."""
    if num_leaves < 1:
        raise ValueError(f"num_leaves must be >= 1, got {num_leaves}")
    n = int(num_leaves)
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
