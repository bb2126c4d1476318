"""Pins the tree-selector oracle (oracle/tree.c via oracle.tree) before the HIP
tree kernels are compared with it.

  * the reference's known answers (tests/test_tree.py:61-76, 116-120 in the
    reference): level counts [5, 3, 2, 1], root range (0, 5), parent ranges
    contain their children, tree_node_counts(7) == [7, 4, 2];
  * merge: float64 restatement of the reference's per-parent merge
    (selector/tree.py:48-76) -- means agree, and the chosen prototypes agree
    wherever the distance order is unambiguous; model-dtype rounding of the
    mean checked against torch's bf16/f16 casts; radix 2 and 3, P = 1..8;
  * candidate scores: float64 MaxSim brute force;
  * traversal: the reference test's full-level traversal
    (tests/test_tree.py:24-41 there: score whole levels with the flat gate,
    keep children of the selected parents) restated in float64 gives the
    same leaf sets wherever no score tie is within rounding; closed forms:
    a beam at least as wide as every level keeps exactly the causal leaves,
    and beam 1 is the greedy root-to-leaf path.
"""
import math

import numpy as np
import pytest
import torch

import oracle.tree as otree
from oracle.selector import round_to
from selector.tree import level_ranges, tree_node_counts


def test_reference_layout_known_answers():
    kb, radix = 5, 2
    counts = otree.level_counts(kb, radix)
    assert counts == [5, 3, 2, 1]
    starts, ends = level_ranges(kb, len(counts) - 1, radix)
    assert starts.tolist() == [0] and ends.tolist() == [5]
    for v in range(len(counts) - 1):
        cs, ce = level_ranges(kb, v, radix)
        ps, pe = level_ranges(kb, v + 1, radix)
        parent = torch.arange(len(cs)) // radix
        assert torch.all(ps[parent] <= cs) and torch.all(ce <= pe[parent])
    assert tree_node_counts(7, radix=2) == [7, 4, 2]
    assert tree_node_counts(7, radix=2, include_root=True) == [7, 4, 2, 1]
    with pytest.raises(ValueError):
        tree_node_counts(0)
    with pytest.raises(ValueError):
        tree_node_counts(5, radix=1)


def test_level_range_table_equals_per_level_ranges():
    # build_key_tree takes every level's ranges from one host-built table.
    from selector.tree import _level_range_table
    for kb, radix in ((5, 2), (2048, 2), (1, 2), (10, 3), (7, 2), (81, 3)):
        table = _level_range_table(kb, radix, "cpu")
        assert len(table) == len(otree.level_counts(kb, radix))
        for v, (starts, ends) in enumerate(table):
            want_s, want_e = level_ranges(kb, v, radix)
            assert torch.equal(starts, want_s) and torch.equal(ends, want_e), (kb, radix, v)


@pytest.mark.parametrize("radix,P,n,D", [(2, 4, 7, 5), (3, 4, 7, 5), (2, 8, 9, 16), (2, 1, 5, 8), (3, 3, 10, 12)])
def test_merge_matches_float64_reference_form(radix, P, n, D):
    rng = np.random.default_rng(radix * 100 + P * 10 + n)
    child = rng.standard_normal((3, n, P, D)).astype(np.float32)
    got = otree.tree_merge(child, radix, "float32")
    ref, dist = otree.merge_reference_f64(child, radix)
    np.testing.assert_allclose(got[:, :, 0], ref[:, :, 0], rtol=1e-6, atol=1e-6)
    checked = 0
    for s in range(child.shape[0]):
        for j in range(got.shape[1]):
            d = np.sort(dist[s, j][np.isfinite(dist[s, j])])[::-1]
            # Unambiguous when consecutive kept distances and the cut are well separated.
            gaps = -np.diff(d[:P]) if P > 1 else np.array([1.0])
            cut = d[P - 2] - d[P - 1] if len(d) >= P and P > 1 else 1.0
            if P > 1 and (gaps.min(initial=1.0) < 1e-4 or cut < 1e-4):
                continue
            np.testing.assert_array_equal(got[s, j, 1:], ref[s, j, 1:].astype(np.float32))
            checked += 1
    assert checked >= got.shape[0] * got.shape[1] // 2


def test_merge_mean_rounds_like_the_model_dtype():
    # Two children whose proto-0 sum and mean are not representable in bf16/f16.
    vals = np.array([1.0078125, 1.015625], np.float32)  # bf16-representable, sum 2.0234375
    child = np.zeros((1, 2, 1, 1), np.float32)
    child[0, :, 0, 0] = vals
    for dtype, tdt in (("bfloat16", torch.bfloat16), ("float16", torch.float16)):
        got = otree.tree_merge(child, 2, dtype)[0, 0, 0, 0]
        summed = torch.tensor(vals, dtype=tdt).sum()
        expect = (summed / torch.tensor(2.0, dtype=tdt)).item()
        assert got == np.float32(expect), (dtype, got, expect)
        assert got == round_to(round_to(np.float32(vals.sum()), dtype) / 2, dtype)


def test_candidate_scores_match_float64_maxsim():
    rng = np.random.default_rng(5)
    S, qb, N, C, Pq, Pk, p = 2, 5, 11, 4, 3, 5, 16
    qp = rng.standard_normal((S, qb, Pq, p)).astype(np.float32)
    kp = rng.standard_normal((S, N, Pk, p)).astype(np.float32)
    ids = rng.integers(-2, N + 2, size=(S, qb, C)).astype(np.int32)
    div = math.sqrt(p)
    got = otree.candidate_scores(qp, kp, ids, div)
    for s in range(S):
        for q in range(qb):
            nodes = np.clip(ids[s, q], 0, N - 1)
            ref = otree.maxsim_f64(qp[s, q], kp[s, nodes], div)
            np.testing.assert_allclose(got[s, q], ref, rtol=2e-6, atol=2e-6)


def _random_tree(seed, S, kb, P, d, p, radix, Pq=None):
    rng = np.random.default_rng(seed)
    Pq = Pq or P
    leaf = rng.standard_normal((S, kb, P, d)).astype(np.float32)
    levels = otree.build_tree(leaf, radix, "float32")
    W = (rng.standard_normal((d, p)) / math.sqrt(d)).astype(np.float32)
    kp_levels = [np.einsum("snkd,dp->snkp", lv.astype(np.float64), W).astype(np.float32) for lv in levels]
    qp = rng.standard_normal((S, kb, Pq, p)).astype(np.float32)
    return qp, kp_levels


@pytest.mark.parametrize("kb,radix,beam", [(13, 2, 3), (16, 2, 2), (20, 3, 2), (33, 2, 5), (7, 2, 1)])
def test_traversal_matches_full_level_reference(kb, radix, beam):
    qp, kp_levels = _random_tree(kb * 7 + beam, 2, kb, 3, 8, 8, radix)
    div = math.sqrt(8)
    got = otree.tree_traverse(qp, np.concatenate(kp_levels, axis=1), kb, radix, beam, div)
    sets, gaps = otree.full_level_traverse_f64(qp, kp_levels, kb, radix, beam, div)
    checked = 0
    for r, (want, gap) in enumerate(zip(sets, gaps)):
        s, q = divmod(r, kb)
        row = got[s, q]
        assert list(row[row < 0]) == [-1] * int((row < 0).sum())
        assert (row[: (row >= 0).sum()] >= 0).all(), "valid IDs come first"
        if gap < 1e-4:
            continue
        assert set(row[row >= 0].tolist()) == want, (s, q)
        checked += 1
    assert checked >= len(sets) * 3 // 4


@pytest.mark.parametrize("kb,radix", [(9, 2), (16, 2), (10, 3)])
def test_wide_beam_keeps_exactly_the_causal_leaves(kb, radix):
    qp, kp_levels = _random_tree(kb, 1, kb, 2, 4, 4, radix)
    beam = 64 // radix
    got = otree.tree_traverse(qp, np.concatenate(kp_levels, axis=1), kb, radix, beam, 2.0)
    for q in range(kb):
        row = got[0, q]
        assert sorted(row[row >= 0].tolist()) == list(range(q + 1)), q


def test_beam_one_is_the_greedy_path():
    kb, radix = 21, 2
    qp, kp_levels = _random_tree(3, 2, kb, 3, 6, 6, radix)
    div = math.sqrt(6)
    got = otree.tree_traverse(qp, np.concatenate(kp_levels, axis=1), kb, radix, 1, div)
    counts = otree.level_counts(kb, radix)
    for s in range(2):
        for q in range(kb):
            node = 0
            for v in range(len(counts) - 2, -1, -1):
                kids = [c for c in range(node * radix, min(node * radix + radix, counts[v]))
                        if c * radix ** v <= q]
                sc = otree.maxsim_f64(qp[s, q], kp_levels[v][s, kids], div)
                node = kids[int(np.argmax(sc))]
            assert got[s, q, 0] == node
