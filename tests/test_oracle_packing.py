"""Pins the route-packing oracle (oracle/packing.py) before it is trusted.

Known answers are the reference's own cases (tests/test_export_selected_blocks.py
in the reference): the 4x4 mask with local priority (:11-27), the narrow-row
error (:30-33), the sink cases (:36-80) and the mask/IDs equivalence (:83-101).
A per-row brute force written from the policy's description (sets, not the
sentinel sort the oracle uses) checks random rows, including duplicates,
out-of-range IDs, kb != qb and sinks.
"""
import numpy as np
import pytest

import oracle.packing as op


def _brute_ids(ids, k, lw, kb, sink):
    L, G, qb, C = ids.shape
    sink = min(sink, kb)
    width = min(k, C + sink + lw + 1)
    out = np.full((1, L, G, qb, width), -1, np.int32)
    for l in range(L):
        for g in range(G):
            for q in range(qb):
                local = [j for j in range(q - lw, q + 1) if j >= 0]
                sinks = [s for s in range(sink) if s < q - lw]
                cand = sorted({int(i) for i in ids[l, g, q] if 0 <= i < kb and sink <= i < q - lw})
                budget = k - len(local) - len(sinks)
                row = sorted(sinks + cand[:budget] + local)
                out[0, l, g, q, : len(row)] = row
    return out


def _brute_mask(mask, k, lw):
    L, G, qb, kb = mask.shape
    out = np.full((1, L, G, qb, min(k, kb)), -1, np.int32)
    for l in range(L):
        for g in range(G):
            for q in range(qb):
                local = [j for j in range(max(0, q - lw), min(q, kb - 1) + 1)]
                cand = [j for j in range(min(q - lw, kb)) if j >= 0 and mask[l, g, q, j]]
                row = sorted(cand[: k - len(local)] + local)
                out[0, l, g, q, : len(row)] = row
    return out


def test_reference_mask_case_local_priority():
    sel = np.zeros((2, 2, 4, 4), bool)
    sel[..., 0, 0] = sel[..., 1, 0] = sel[..., 2, 0] = sel[..., 3, 0] = sel[..., 3, 1] = True
    packed = op.pack_mask(sel, k_selected=3, local_window=1)
    assert packed.shape == (1, 2, 2, 4, 3)
    assert packed[0, 0, 0].tolist() == [[0, -1, -1], [0, 1, -1], [0, 1, 2], [0, 2, 3]]
    assert np.array_equal(packed, _brute_mask(sel, 3, 1))


def test_reference_errors():
    with pytest.raises(ValueError, match="cannot fit local window"):
        op.pack_mask(np.ones((1, 1, 3, 3), bool), k_selected=1, local_window=1)
    with pytest.raises(ValueError, match="sink block"):
        op.pack_ids(np.zeros((1, 1, 4, 2), np.int64), k_selected=2, local_window=1, key_blocks=4, sink_blocks=1)


def test_reference_sink_cases():
    ids = np.array([[[[0, -1], [1, 0], [0, 2], [1, 3]]]])
    assert np.array_equal(op.pack_ids(ids, 3, 1, 4), op.pack_ids(ids, 3, 1, 4, sink_blocks=0))
    ids = np.array([[[[5, 5], [5, 5], [5, 5], [2, 5], [2, 3], [3, 4]]]])
    assert 0 not in op.pack_ids(ids, 4, 1, 6)[0, 0, 0, 5].tolist()
    with_sink = op.pack_ids(ids, 4, 1, 6, sink_blocks=1)
    assert all(with_sink[0, 0, 0, r, 0] == 0 for r in range(6))
    packed = op.pack_ids(np.full((1, 1, 4, 2), -1), 3, 1, 4, sink_blocks=1)
    assert packed[0, 0, 0, 0].tolist() == [0, -1, -1]
    assert packed[0, 0, 0, 1].tolist() == [0, 1, -1]


def test_reference_ids_match_mask_policy():
    ids = np.array([[[[0, -1, -1], [1, 0, -1], [0, 2, 1], [1, 0, 3]]]])
    with_pad = np.zeros((1, 1, 4, 5), bool)
    safe = np.where(ids < 0, 4, ids)
    for q in range(4):
        with_pad[0, 0, q, safe[0, 0, q]] = True
    assert np.array_equal(op.pack_ids(ids, 3, 1, 4), op.pack_mask(with_pad[..., :4], 3, 1))


@pytest.mark.parametrize("seed,qb,kb,C,k,lw,sink", [
    (0, 9, 9, 5, 4, 1, 0), (1, 12, 7, 8, 6, 2, 1), (2, 6, 11, 3, 8, 0, 3),
    (3, 20, 20, 16, 5, 1, 2), (4, 5, 5, 1, 2, 1, 0), (5, 15, 40, 30, 12, 3, 4),
])
def test_oracle_matches_brute_force(seed, qb, kb, C, k, lw, sink):
    rng = np.random.default_rng(seed)
    ids = rng.integers(-3, max(qb, kb) + 3, size=(2, 3, qb, C))
    assert np.array_equal(op.pack_ids(ids, k, lw, kb, sink), _brute_ids(ids, k, lw, kb, sink))
    mask = rng.random((2, 3, qb, kb)) < 0.3
    if k >= lw + 1:
        assert np.array_equal(op.pack_mask(mask, k, lw), _brute_mask(mask, k, lw))
