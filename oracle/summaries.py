"""CPU oracle for the residual-tree summaries -- TEST INFRASTRUCTURE ONLY.

Only tests/ use this module, as the checker of the HIP summary kernels.

Restatements (numpy, float64):
  tree_layout     build_residual_tree_layout (interfaces/residual_summaries.py:72-116):
                  level counts ceil(prev / 2); each node's leaf range is the
                  union of its children's ranges, built level by level.
  token_ranges    _prototype_token_ranges (sparse/summaries.py:29-49).
  kv_summary      build_kv_summary_table (sparse/summaries.py:52-142): per
                  range the mean of the valid rows (sum / max(count, 1)),
                  count, log(count) or -inf.  Direct float64 sums.
  prefix_summary  the same table by the reference's own method (differences
                  of prefix sums, :105-122), used to cross-check kv_summary.
  frontier_visit  residual_frontier_for_row (interfaces/residual_summaries.py:
                  119-147): the top-down visit from the root that keeps a node
                  when its range is causal and holds no listed block, else
                  recurses into its children; sorted by node ID.
  frontier_dyadic an independent construction of the same set: every gap
                  between listed blocks, cut greedily from its left end into
                  the largest tree node that starts there and fits.

Pinned by tests/test_oracle_summaries.py: the reference's known answers
(tests/test_residual_summaries.py:25-41 and tests/test_summary_pooling.py:49-88
in the reference) and the agreement of the two summation methods.  The two
frontier constructions are pinned by the reference's frontier known answers
(tests/test_residual_summaries.py:44-64 there), by agreeing with each other,
and by the partition and maximality properties checked from first principles
(tests/test_oracle_frontier.py).
"""
import numpy as np


def tree_layout(num_leaves):
    """-> dict(level_counts, level_offsets, starts, ends, levels, indices) as tuples."""
    if num_leaves < 1:
        raise ValueError(f"num_leaves must be >= 1, got {num_leaves}")
    counts = [num_leaves]
    while counts[-1] > 1:
        counts.append((counts[-1] + 1) // 2)
    offsets = list(np.cumsum([0] + counts[:-1]))
    starts, ends, levels, indices = [], [], [], []
    prev = None
    for level, count in enumerate(counts):
        if level == 0:
            cur = [(i, i + 1) for i in range(count)]
        else:
            cur = [(prev[2 * i][0], prev[min(2 * i + 1, len(prev) - 1)][1]) for i in range(count)]
        for i, (s, e) in enumerate(cur):
            starts.append(s)
            ends.append(e)
            levels.append(level)
            indices.append(i)
        prev = cur
    return dict(level_counts=tuple(counts), level_offsets=tuple(int(o) for o in offsets),
                starts=tuple(starts), ends=tuple(ends), levels=tuple(levels), indices=tuple(indices))


def token_ranges(starts, ends, seq_len, block_size, prototypes):
    first = np.minimum(np.asarray(starts, np.int64) * block_size, seq_len)
    last = np.minimum(np.asarray(ends, np.int64) * block_size, seq_len)
    length = (last - first)[:, None]
    p = np.arange(prototypes)[None, :]
    return first[:, None] + length * p // prototypes, first[:, None] + length * (p + 1) // prototypes


def kv_summary(key, value, rs, re, valid=None):
    """key/value [B,H,T,D]; rs/re [N,P] token ranges; valid [B,T] bool or None.
    Returns keys, values [B,H,N,P,D], counts, log_counts [B,N,P] (float64)."""
    key = np.asarray(key, np.float64)
    value = np.asarray(value, np.float64)
    B, H, T, D = key.shape
    w = np.ones((B, T)) if valid is None else np.asarray(valid, np.float64)
    N, P = rs.shape
    keys = np.zeros((B, H, N, P, D))
    vals = np.zeros((B, H, N, P, D))
    counts = np.zeros((B, N, P))
    for n in range(N):
        for p in range(P):
            s, e = int(rs[n, p]), int(re[n, p])
            c = w[:, s:e].sum(axis=1)
            counts[:, n, p] = c
            den = np.maximum(c, 1.0)[:, None, None]
            keys[:, :, n, p] = (key[:, :, s:e] * w[:, None, s:e, None]).sum(axis=2) / den
            vals[:, :, n, p] = (value[:, :, s:e] * w[:, None, s:e, None]).sum(axis=2) / den
    with np.errstate(divide="ignore"):
        logc = np.where(counts > 0, np.log(np.maximum(counts, 1e-300)), -np.inf)
    return keys, vals, counts, logc


def prefix_summary(key, value, rs, re, valid=None):
    """The same table from prefix-sum differences (the reference's method)."""
    key = np.asarray(key, np.float64)
    value = np.asarray(value, np.float64)
    B, H, T, D = key.shape
    w = np.ones((B, T)) if valid is None else np.asarray(valid, np.float64)
    N, P = rs.shape
    fs, fe = rs.reshape(-1), re.reshape(-1)

    def pool(x):
        pre = np.concatenate([np.zeros((B, H, 1, D)), np.cumsum(x * w[:, None, :, None], axis=2)], axis=2)
        return (pre[:, :, fe] - pre[:, :, fs]).reshape(B, H, N, P, D)

    cpre = np.concatenate([np.zeros((B, 1)), np.cumsum(w, axis=1)], axis=1)
    counts = (cpre[:, fe] - cpre[:, fs]).reshape(B, N, P)
    den = np.maximum(counts, 1.0)[:, None, :, :, None]
    with np.errstate(divide="ignore"):
        logc = np.where(counts > 0, np.log(np.maximum(counts, 1e-300)), -np.inf)
    return pool(key) / den, pool(value) / den, counts, logc


def frontier_visit(selected, qb, layout):
    """Maximal tree nodes covering the causal blocks [0, qb] not in `selected`.

    layout: the dict of tree_layout().  Raises ValueError for a listed id > qb,
    as the reference does."""
    listed = sorted({int(b) for b in selected if int(b) >= 0})
    if listed and listed[-1] > qb:
        raise ValueError("selected block IDs must be causal and non-negative")
    starts, ends, levels, indices = (layout[f] for f in ("starts", "ends", "levels", "indices"))
    counts, offsets = layout["level_counts"], layout["level_offsets"]
    listed_set = set(listed)
    out = []

    def visit(node):
        s, e = starts[node], ends[node]
        if s > qb:
            return
        if e <= qb + 1 and not any(j in listed_set for j in range(s, e)):
            out.append(node)
            return
        lvl = levels[node]
        if lvl == 0:
            return
        for c in (2 * indices[node], 2 * indices[node] + 1):
            if c < counts[lvl - 1]:
                visit(offsets[lvl - 1] + c)

    visit(offsets[-1])
    return sorted(out)


def frontier_dyadic(selected, qb, num_leaves):
    """Same set by greedy decomposition of each gap [a, b) between listed blocks.

    From a, take the highest-level node that starts at a (a divisible by its
    width) and ends (clipped to num_leaves) at or before b; repeat from its
    end.  Node (level v, index i) has ID sum of the level counts below v, + i."""
    listed = sorted({int(b) for b in selected if 0 <= int(b) <= qb})
    counts = [num_leaves]
    while counts[-1] > 1:
        counts.append((counts[-1] + 1) // 2)
    offsets = [sum(counts[:v]) for v in range(len(counts))]
    gaps, prev = [], -1
    for j in listed + [qb + 1]:
        if j > prev + 1:
            gaps.append((prev + 1, j))
        prev = j
    out = []
    for a, b in gaps:
        pos = a
        while pos < b:
            v = 0
            while (v + 1 < len(counts) and pos % (1 << (v + 1)) == 0
                   and min(pos + (1 << (v + 1)), num_leaves) <= b):
                v += 1
            out.append(offsets[v] + (pos >> v))
            pos = min(pos + (1 << v), num_leaves)
    return sorted(out)
