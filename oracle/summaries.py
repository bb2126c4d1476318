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

Pinned by tests/test_oracle_summaries.py: the reference's known answers
(tests/test_residual_summaries.py:25-41 and tests/test_summary_pooling.py:49-88
in the reference) and the agreement of the two summation methods.
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
