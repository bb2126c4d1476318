"""Pins the selector oracle (oracle/selector.c) before it is trusted.

Known answers from the reference's own tests (group average,
tests/test_group_avg.py:6-13; block mean and ragged block,
tests/test_proto_pool.py:7-14,57-67; brute-force MaxSim,
tests/test_gate_maxsim.py:22-33; stable descending top-k,
selector/baselines.py:59-62), closed forms that are exact in float32
(integer-valued inputs), and deliberate ties for the lowest-index rule.
"""
import math

import numpy as np
import pytest

import oracle.selector as osel


def test_group_average_and_block_mean_match_reference_semantics():
    # Reference: x.view(b, G, H/G, L, d).mean(dim=2) per token, then the block mean.
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 12, 10, 8)).astype(np.float32)       # G = 2 groups of 6 heads
    k = rng.standard_normal((1, 2, 10, 8)).astype(np.float32)
    q_mean, k_sum = osel.block_pool(x, k)
    grouped = x.astype(np.float64).reshape(1, 2, 6, 10, 8).mean(axis=2)   # [1,2,10,8]
    np.testing.assert_allclose(q_mean[0, :, 0], grouped[0].mean(axis=1), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(k_sum[0, :, 0, 0], k[0].astype(np.float64).mean(axis=1), rtol=1e-6, atol=1e-6)


def test_full_and_ragged_block_means_and_exact_max():
    rng = np.random.default_rng(1)
    T = 64 + 3                                                      # last block has 3 real rows
    k = rng.standard_normal((1, 1, T, 16)).astype(np.float32)
    _, k_sum = osel.block_pool(None, k)
    np.testing.assert_allclose(k_sum[0, 0, 0, 0], k[0, 0, :64].mean(axis=0), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(k_sum[0, 0, 1, 0], k[0, 0, 64:].mean(axis=0), rtol=1e-6, atol=1e-6)
    assert np.array_equal(k_sum[0, 0, 0, 1], k[0, 0, :64].max(axis=0))
    assert np.array_equal(k_sum[0, 0, 1, 1], k[0, 0, 64:].max(axis=0))   # pad rows never win


@pytest.mark.parametrize("D", [8, 16, 80, 96, 120, 128, 200, 264, 1000, 2048])
def test_block_mean_and_max_match_plain_block_statistics(D):
    # The lane layout must cover all 64 tokens of a block at every head_dim the
    # ABI accepts (multiples of 8 up to 2048), not only powers of two: the
    # float32 means agree with float64 block means to rounding, the maxima exactly.
    rng = np.random.default_rng(D)
    T, G = 64 * 2 + 37, 3
    q = rng.standard_normal((1, G, T, D)).astype(np.float32)
    k = rng.standard_normal((1, 1, T, D)).astype(np.float32)
    q_mean, k_sum = osel.block_pool(q, k)
    for blk, (a, b) in enumerate(((0, 64), (64, 128), (128, T))):
        qm = q[0, :, a:b].astype(np.float64).mean(axis=(0, 1))
        km = k[0, 0, a:b].astype(np.float64).mean(axis=0)
        np.testing.assert_allclose(q_mean[0, 0, blk], qm, rtol=0, atol=2e-6)
        np.testing.assert_allclose(k_sum[0, 0, blk, 0], km, rtol=0, atol=2e-6)
        assert np.array_equal(k_sum[0, 0, blk, 1], k[0, 0, a:b].max(axis=0))


def test_integer_valued_pooling_and_projection_are_exact():
    # Small integers: every sum is exact, so only the final division rounds.
    rng = np.random.default_rng(2)
    q = rng.integers(-8, 9, size=(1, 7, 130, 128)).astype(np.float32)
    k = rng.integers(-8, 9, size=(1, 1, 130, 128)).astype(np.float32)
    q_mean, k_sum = osel.block_pool(q, k)
    for blk, (a, b) in enumerate(((0, 64), (64, 128), (128, 130))):
        s = q[0, :, a:b].astype(np.float64).sum(axis=(0, 1))
        expect = (s.astype(np.float32) / np.float32(7 * (b - a))).astype(np.float32)
        assert np.array_equal(q_mean[0, 0, blk], expect)
    W = rng.integers(-4, 5, size=(128, 128)).astype(np.float32)
    x = rng.integers(-4, 5, size=(5, 128)).astype(np.float32)
    assert np.array_equal(osel.project(x, W), (x.astype(np.int64) @ W.astype(np.int64)).astype(np.float32))


def test_scores_match_bruteforce_maxsim():
    # Reference tests/test_gate_maxsim.py:22-33: project, all prototype pairs, max, / sqrt(p).
    rng = np.random.default_rng(3)
    G, qb, kb, Pq, Pk, d, p = 2, 5, 5, 2, 3, 8, 6
    qf = rng.standard_normal((G, qb, Pq, d)).astype(np.float32)
    kf = rng.standard_normal((G, kb, Pk, d)).astype(np.float32)
    Wq = rng.standard_normal((d, p)).astype(np.float32)
    Wk = rng.standard_normal((d, p)).astype(np.float32)
    qp, kp = osel.project(qf, Wq), osel.project(kf, Wk)
    s = osel.scores(qp, kp)
    qp64 = np.einsum("gqid,dp->gqip", qf.astype(np.float64), Wq.astype(np.float64))
    kp64 = np.einsum("gkjd,dp->gkjp", kf.astype(np.float64), Wk.astype(np.float64))
    ref = np.einsum("gqip,gkjp->gqkij", qp64, kp64).max(axis=(-1, -2)) / math.sqrt(p)
    causal = np.tril(np.ones((qb, kb), bool))
    np.testing.assert_allclose(s[:, causal], ref[:, causal], rtol=1e-5, atol=1e-5)
    assert np.all(np.isneginf(s[:, ~causal]))


def test_topk_is_stable_descending_with_lowest_index_ties():
    rng = np.random.default_rng(4)
    R, Qb, k = 3, 40, 8
    s = rng.standard_normal((R, Qb, Qb)).astype(np.float32)
    s[0, 30, :31] = 1.0                        # a row of ties: lowest 8 indices win
    s[1, 20, [3, 9, 17]] = 5.0                 # tied maxima
    out = osel.topk(s, k)
    for r in range(R):
        for i in range(Qb):
            n = min(i + 1, Qb)
            order = np.argsort(-s[r, i, :n], kind="stable")[:k]
            expect = np.sort(order)
            got = out[r, i]
            assert np.array_equal(got[: len(expect)], expect), (r, i)
            assert np.all(got[len(expect):] == -1)
    assert out[0, 30].tolist() == list(range(8))
    assert out[0, 3].tolist() == [0, 1, 2, 3, -1, -1, -1, -1]     # short causal row


def test_flat_select_shapes_and_contract():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 4, 300, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, 300, 64)).astype(np.float32)
    Wq = rng.standard_normal((64, 64)).astype(np.float32)
    Wk = rng.standard_normal((64, 64)).astype(np.float32)
    out = osel.flat_select(q, k, Wq, Wk, top_k=3)
    sel = out["selected"]
    assert sel.shape == (1, 1, 2, 5, 3) and sel.dtype == np.int32
    for g in range(2):
        for i in range(5):
            row = [x for x in sel[0, 0, g, i] if x >= 0]
            assert row == sorted(set(row)) and all(0 <= x <= i for x in row)
            assert len(row) == min(3, i + 1)
