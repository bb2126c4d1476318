"""Pins the residual-summary oracle (oracle/summaries.py) and the host tree layout.

Known answers: the reference's layout cases (tests/test_residual_summaries.py:25-41
in the reference) and summary-pooling cases (tests/test_summary_pooling.py:49-88).
The host layout (closed-form ranges) must equal the oracle's level-by-level
construction for every leaf count up to 300; the oracle's direct sums must
equal the reference's prefix-difference method.
"""
import math

import numpy as np
import pytest

import oracle.summaries as osum
from interfaces.residual_summaries import build_residual_tree_layout


def test_reference_layout_cases():
    lay = build_residual_tree_layout(5)
    assert lay.level_counts == (5, 3, 2, 1)
    assert lay.level_offsets == (0, 5, 8, 10)
    assert lay.num_nodes == 11
    assert lay.range(5) == (0, 2) and lay.range(7) == (4, 5) and lay.range(9) == (4, 5)
    assert lay.range(lay.root_id) == (0, 5)
    assert lay.children(lay.root_id) == (8, 9)
    for n in (256, 512, 1024, 2048):
        lay = build_residual_tree_layout(n)
        assert lay.range(lay.root_id) == (0, n) and lay.num_nodes == 2 * n - 1
    with pytest.raises(ValueError):
        build_residual_tree_layout(0)


def test_host_layout_equals_oracle_construction():
    for n in range(1, 301):
        lay = build_residual_tree_layout(n)
        ref = osum.tree_layout(n)
        for field, val in ref.items():
            assert getattr(lay, field) == val, (n, field)
        for node in range(lay.num_nodes):
            kids = lay.children(node)
            if kids:
                assert (lay.starts[kids[0]], lay.ends[kids[-1]]) == lay.range(node)


def _table(key, value, n_leaves, block_size, P, valid=None):
    lay = osum.tree_layout(n_leaves)
    rs, re = osum.token_ranges(lay["starts"], lay["ends"], key.shape[2], block_size, P)
    return osum.kv_summary(key, value, rs, re, valid)


def test_reference_pooling_means_counts_and_empty_tail_prototype():
    key = np.arange(5, dtype=np.float64).reshape(1, 1, 5, 1)
    keys, vals, counts, logc = _table(key, key * 10, 3, 2, 2)
    assert counts[0, 3].tolist() == [2.0, 2.0]
    assert keys[0, 0, 3, :, 0].tolist() == [0.5, 2.5]
    assert vals[0, 0, 3, :, 0].tolist() == [5.0, 25.0]
    np.testing.assert_allclose(logc[0, 3], [math.log(2.0)] * 2)
    assert counts[0, 2].tolist() == [0.0, 1.0]
    assert np.isneginf(logc[0, 2, 0]) and keys[0, 0, 2, 1, 0] == 4.0


def test_reference_padding_tokens_do_not_contribute():
    key = np.array([100.0, 100.0, 2.0, 4.0]).reshape(1, 1, 4, 1)
    valid = np.array([[False, False, True, True]])
    keys, _, counts, _ = _table(key, key, 2, 2, 1, valid)
    root = 2
    assert counts[0, root, 0] == 2 and keys[0, 0, root, 0, 0] == 3.0


@pytest.mark.parametrize("T,bs,P", [(37, 4, 4), (64, 8, 2), (129, 16, 1)])
def test_direct_sums_equal_prefix_method(T, bs, P):
    rng = np.random.default_rng(T)
    key = rng.standard_normal((2, 3, T, 5))
    value = rng.standard_normal((2, 3, T, 5))
    valid = rng.random((2, T)) < 0.8
    lay = osum.tree_layout((T + bs - 1) // bs)
    rs, re = osum.token_ranges(lay["starts"], lay["ends"], T, bs, P)
    a = osum.kv_summary(key, value, rs, re, valid)
    b = osum.prefix_summary(key, value, rs, re, valid)
    for x, y in zip(a, b):
        np.testing.assert_allclose(x, y, atol=1e-12)
