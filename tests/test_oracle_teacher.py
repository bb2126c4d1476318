"""Pins the teacher oracle (oracle/teacher.py) before it is trusted.

block_mass must equal pool_attention of an independent dense causal softmax
(the reference's own integration check compares chunked_pool with
pool_attention, tests/validate_chunked_extract.py:24-54 in the reference),
and satisfy the invariants the mathematics fixes: rows sum to the number of
real query rows, the upper triangle is exactly zero (check_causal), rollup
preserves totals, normalised targets rows sum to one.
"""
import numpy as np
import pytest

import oracle.teacher as ot


@pytest.mark.parametrize("T,H,Hkv,D,block", [(20, 4, 2, 8, 4), (150, 3, 1, 16, 64), (7, 2, 2, 4, 2)])
def test_block_mass_equals_pooled_dense_attention(T, H, Hkv, D, block):
    rng = np.random.default_rng(T)
    q = rng.standard_normal((1, H, T, D))
    k = rng.standard_normal((1, Hkv, T, D))
    mass = ot.block_mass(q, k, block=block)
    ref = ot.pool_attention(ot.dense_causal_softmax(q, k), block)
    np.testing.assert_allclose(mass, ref, atol=1e-12)


def test_invariants_rows_causality_rollup_targets():
    rng = np.random.default_rng(1)
    T, block = 100, 8                                      # 13 blocks, last one ragged (4 rows)
    q = rng.standard_normal((2, 4, T, 8))
    k = rng.standard_normal((2, 2, T, 8))
    mass = ot.block_mass(q, k, block=block)
    rows = np.full(13, 8.0)
    rows[-1] = T - 12 * 8
    np.testing.assert_allclose(mass.sum(axis=-1), np.broadcast_to(rows, mass.shape[:-1]), atol=1e-9)
    ok, where = ot.check_causal(mass)
    assert ok and where is None
    assert np.all(np.triu(mass, k=1) == 0)
    lv = ot.rollup(mass[:, :, :12, :12])
    assert [x.shape[-1] for x in lv] == [12, 6, 3]
    for a in lv[1:]:
        np.testing.assert_allclose(a.sum(axis=(-1, -2)), lv[0].sum(axis=(-1, -2)))
    target, row_mass, top = ot.targets(mass, 2, k=3)
    np.testing.assert_allclose(target.sum(axis=-1), 1.0, atol=1e-12)
    np.testing.assert_allclose(row_mass, mass.reshape(2, 2, 2, 13, 13).mean(axis=2).sum(-1))
    assert top[0, 0, 0].tolist() == [0, -1, -1]
    order = np.argsort(-target[1, 1, 9, :10], kind="stable")[:3]
    assert top[1, 1, 9].tolist() == order.tolist()


def test_check_causal_detects_leak():
    pooled = np.zeros((1, 1, 3, 3))
    pooled[0, 0, 1, 2] = 1e-3
    assert ot.check_causal(pooled) == (False, (1, 2))
