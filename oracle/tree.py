"""Tree-selector oracle (ctypes wrapper of oracle/tree.c) -- TEST INFRASTRUCTURE ONLY.

tree.c fixes the float32 operation order of the HIP tree kernels, so merged
node prototypes, candidate scores and the traversed leaf IDs compare bit for
bit.  Reference semantics (file:line) are listed in oracle/tree.c.  Besides
the C restatement this module holds an independent float64 form of the
reference's own algorithms (per-parent merge of selector/tree.py:48-76 and
the full-level traversal of the reference's tests/test_tree.py:24-41), used
to pin tree.c.
"""
import ctypes
import math

import numpy as np

from oracle.selector import DTYPE_CODES, lib as _selector_lib

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_ready = False


def _lib():
    global _ready
    h = _selector_lib()
    if not _ready:
        ci = ctypes.c_int
        h.oracle_tree_merge.argtypes = [_f32p, ci, ci, ci, ci, ci, ci, _f32p]
        h.oracle_tree_merge.restype = None
        h.oracle_candidate_scores.argtypes = [_f32p, _f32p, _i32p, ci, ci, ci, ci, ci, ci, ci,
                                              ctypes.c_float, _f32p]
        h.oracle_candidate_scores.restype = None
        h.oracle_tree_traverse.argtypes = [_f32p, _f32p, ci, ci, ci, ci, ci, ci, ci, ci, ci,
                                           ctypes.c_float, _i32p]
        h.oracle_tree_traverse.restype = ci
        _ready = True
    return h


def level_counts(kb, radix):
    counts = [kb]
    while counts[-1] > 1:
        counts.append((counts[-1] + radix - 1) // radix)
    return counts


def tree_merge(child, radix, dtype):
    """child [S, n, P, D] model-dtype values (float32) -> parent [S, ceil(n/radix), P, D]."""
    child = np.ascontiguousarray(child, dtype=np.float32)
    S, n, P, D = child.shape
    m = (n + radix - 1) // radix
    out = np.zeros((S, m, P, D), np.float32)
    _lib().oracle_tree_merge(child, S, n, P, D, radix, DTYPE_CODES[dtype], out)
    return out


def build_tree(leaf, radix, dtype):
    """All levels leaf-first: [leaf, level 1, ..., root], each [S, n_v, P, D]."""
    levels = [np.ascontiguousarray(leaf, dtype=np.float32)]
    while levels[-1].shape[1] > 1:
        levels.append(tree_merge(levels[-1], radix, dtype))
    return levels


def candidate_scores(qp, kp, ids, div):
    qp = np.ascontiguousarray(qp, dtype=np.float32)
    kp = np.ascontiguousarray(kp, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    S, qb, Pq, pd = qp.shape
    N, Pk = kp.shape[1], kp.shape[2]
    C = ids.shape[2]
    out = np.zeros((S, qb, C), np.float32)
    _lib().oracle_candidate_scores(qp, kp, ids, S, qb, N, C, Pq, Pk, pd, float(div), out)
    return out


def tree_traverse(qp, kp_all, kb, radix, beam, div, q0=0):
    """qp [S, nq, Pq, p] for query blocks q0..q0+nq-1; kp_all [S, N, Pk, p]
    (all levels, leaf-first) -> [S, nq, C] int32."""
    qp = np.ascontiguousarray(qp, dtype=np.float32)
    kp_all = np.ascontiguousarray(kp_all, dtype=np.float32)
    S, qb, Pq, pd = qp.shape
    Pk = kp_all.shape[2]
    W = 1
    counts = level_counts(kb, radix)
    for n in reversed(counts[:-1]):
        W = min(beam, W * radix, n)
    out = np.zeros((S, qb, W), np.int32)
    C = _lib().oracle_tree_traverse(qp, kp_all, S, q0, qb, kb, Pq, Pk, pd, radix, beam, float(div), out)
    assert C == W
    return out


# ---------------------------------------------------------------- float64 forms

def merge_reference_f64(child, radix):
    """Per-parent merge in float64 following selector/tree.py:48-76: mean of
    the children's prototype 0; the P-1 candidates farthest from it.
    Returns (parent [S, m, P, D], dist [S, m, radix*P] with -inf for missing
    children) so callers can tell unambiguous choices."""
    child = np.asarray(child, dtype=np.float64)
    S, n, P, D = child.shape
    m = (n + radix - 1) // radix
    parent = np.zeros((S, m, P, D))
    dists = np.full((S, m, radix * P), -np.inf)
    for s in range(S):
        for j in range(m):
            kids = child[s, j * radix:min((j + 1) * radix, n)]
            mean = kids[:, 0].mean(axis=0)
            cand = kids.reshape(-1, D)
            d = ((cand - mean) ** 2).sum(axis=1)
            dists[s, j, :len(d)] = d
            parent[s, j, 0] = mean
            order = np.argsort(-d, kind="stable")[:P - 1]
            parent[s, j, 1:1 + len(order)] = cand[order]
    return parent, dists


def maxsim_f64(qp, kp_nodes, div):
    """qp [Pq, p], kp_nodes [M, Pk, p] -> [M] max over prototype pairs / div (float64)."""
    s = np.einsum("ap,mcp->mac", np.asarray(qp, np.float64), np.asarray(kp_nodes, np.float64))
    return s.reshape(s.shape[0], -1).max(axis=1) / div


def full_level_traverse_f64(qp, kp_levels, kb, radix, beam, div):
    """The reference test's full-level traversal (tests/test_tree.py:24-41):
    at each level score every node, keep the children of the selected parents
    that start at or before the query block, take the top min(beam, level
    nodes).  Returns per row the leaf selection as a set, plus the smallest
    score gap met at any cut (for unambiguous comparison)."""
    counts = level_counts(kb, radix)
    S, qb = qp.shape[:2]
    rows, gaps = [], []
    for s in range(S):
        for q in range(qb):
            selected = {0}
            gap = math.inf
            for v in range(len(counts) - 2, -1, -1):
                n = counts[v]
                span = radix ** v
                cand = [c for c in range(n) if c // radix in selected and c * span <= q]
                sc = maxsim_f64(qp[s, q], kp_levels[v][s], div)
                k = min(beam, n)
                order = sorted(cand, key=lambda c: (-sc[c], c))
                if len(order) > k:
                    gap = min(gap, sc[order[k - 1]] - sc[order[k]])
                selected = set(order[:k])
            rows.append(selected)
            gaps.append(gap)
    return rows, gaps
