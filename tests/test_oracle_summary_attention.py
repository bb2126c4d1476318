"""Pins the residual-summary attention oracle (oracle.attention.sparse_attention_summaries).

  * The reference's known answers (tests/test_summary_pooling.py:91-121 and
    :176-207 in the reference): with identical keys, the log(count)
    multiplicity bias makes exact blocks + summaries equal dense causal
    attention for P = 1, 2, 4; an all-blocks route has an empty frontier and
    stays equal to dense attention.
  * A pure-Python brute force (scalar loops, math.exp, float64) that builds
    each query's softmax set explicitly -- causal exact keys, then one entry
    per non-empty node prototype with its log(count) -- on random GQA inputs
    with a ragged last block; catches a dropped bias, a wrong prototype or
    node index, a causal mask applied to summaries, or a wrong head mapping.
"""
import math

import numpy as np
import pytest
import torch

import oracle.summaries as osum
from oracle.attention import dense_causal_attention, sparse_attention_index, sparse_attention_summaries


def _local_routes(qblocks):
    sel = np.full((1, 1, qblocks, 2), -1, np.int32)
    for q in range(qblocks):
        row = list(range(max(0, q - 1), q + 1))
        sel[0, 0, q, : len(row)] = row
    return sel


def _frontier(sel):
    """[B,G,Q,K] routes -> [B,G,Q,S] residual nodes (oracle frontier)."""
    B, G, Q, _ = sel.shape
    lay = osum.tree_layout(Q)
    rows = [[osum.frontier_visit(sel[b, g, q].tolist(), q, lay) for q in range(Q)]
            for b in range(B) for g in range(G)]
    width = max([len(r) for rr in rows for r in rr] + [0])
    out = np.full((B, G, Q, width), -1, np.int32)
    for i, rr in enumerate(rows):
        b, g = divmod(i, G)
        for q, r in enumerate(rr):
            out[b, g, q, : len(r)] = r
    return out


def _table(k, v, qblocks, block_size, P, valid=None):
    lay = osum.tree_layout(qblocks)
    rs, re = osum.token_ranges(lay["starts"], lay["ends"], k.shape[2], block_size, P)
    keys, vals, _, logc = osum.kv_summary(k, v, rs, re, valid)
    N = len(lay["starts"])
    B, H, _, D = k.shape
    return (keys.reshape(B, H, N, P, D), vals.reshape(B, H, N, P, D), logc.reshape(B, N, P))


@pytest.mark.parametrize("prototypes", [1, 2, 4])
def test_reference_kat_identical_keys_match_dense(prototypes):
    torch.manual_seed(4)
    length = 6
    query = torch.randn(1, 2, length, 3).numpy()
    key = np.ones((1, 1, length, 3), np.float32)
    value = np.arange(length * 3, dtype=np.float32).reshape(1, 1, length, 3)
    sel = _local_routes(3)
    nodes = _frontier(sel)
    assert nodes[0, 0].tolist() == [[-1], [-1], [0]]
    sk, sv, sl = _table(key, value, 3, 2, prototypes)
    out = sparse_attention_summaries(query, key, value, sel, nodes, sk, sv, sl, block_size=2)
    np.testing.assert_allclose(out, dense_causal_attention(query, key, value), atol=1e-5, rtol=1e-5)
    # Without summaries the omitted block 0 is simply missing.
    plain = sparse_attention_index(query, key, value, sel, block_size=2)
    assert np.abs(plain - out).max() > 0.1


def test_reference_kat_all_blocks_have_empty_frontier():
    torch.manual_seed(9)
    query = torch.randn(1, 2, 5, 3).numpy()
    key = torch.randn(1, 1, 5, 3).numpy()
    value = torch.randn(1, 1, 5, 3).numpy()
    sel = np.full((1, 1, 3, 3), -1, np.int32)
    for q in range(3):
        sel[0, 0, q, : q + 1] = np.arange(q + 1)
    nodes = _frontier(sel)
    assert nodes.shape[-1] == 0
    sk, sv, sl = _table(key, value, 3, 2, 4)
    out = sparse_attention_summaries(query, key, value, sel, nodes, sk, sv, sl, block_size=2)
    np.testing.assert_allclose(out, dense_causal_attention(query, key, value), atol=1e-5, rtol=1e-5)
    np.testing.assert_array_equal(out, sparse_attention_index(query, key, value, sel, block_size=2))


def _bruteforce(q, k, v, sel, nodes, table_keys, table_vals, table_logc, block_size, valid=None):
    q, k, v = (np.asarray(x, np.float64).tolist() for x in (q, k, v))
    B, Hq, T, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    G = Hq // len(k[0])
    sc = 1.0 / math.sqrt(D)
    out = np.zeros((B, T, Hq, D))
    for b in range(B):
        for h in range(Hq):
            g = h // G
            for t in range(T):
                qb = t // block_size
                entries = []  # (key vector, value vector, additive bias)
                for blk in sel[b, g, qb]:
                    if 0 <= blk <= qb:
                        for j in range(blk * block_size, min((blk + 1) * block_size, T)):
                            if j <= t and (valid is None or valid[b, j]):
                                entries.append((k[b][g][j], v[b][g][j], 0.0))
                for node in nodes[b, g, qb]:
                    if node < 0:
                        continue
                    for p in range(table_keys.shape[3]):
                        bias = float(table_logc[b, node, p])
                        if bias == -math.inf:
                            continue
                        entries.append((table_keys[b, g, node, p].tolist(),
                                        table_vals[b, g, node, p].tolist(), bias))
                if not entries:   # a padding position with nothing to attend
                    continue
                scores = [sum(q[b][h][t][d] * kk[d] for d in range(D)) * sc + bias
                          for kk, _, bias in entries]
                mx = max(scores)
                w = [math.exp(s - mx) for s in scores]
                z = sum(w)
                for d in range(D):
                    out[b, t, h, d] = sum(wi * vv[d] for wi, (_, vv, _) in zip(w, entries)) / z
    return out


@pytest.mark.parametrize("prototypes", [1, 2, 4])
def test_bruteforce_random_gqa_ragged(prototypes):
    rng = np.random.default_rng(prototypes)
    B, Hq, Hkv, T, D, bs = 2, 4, 2, 23, 4, 3
    Q = (T + bs - 1) // bs
    q = rng.standard_normal((B, Hq, T, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    sel = np.full((B, Hkv, Q, 5), -1, np.int32)
    for b, g, qb in np.ndindex(B, Hkv, Q):
        extra = rng.choice(qb + 1, size=min(qb + 1, 2), replace=False).tolist()
        row = sorted(set(extra) | {qb, max(0, qb - 1)})
        sel[b, g, qb, : len(row)] = row
    nodes = _frontier(sel)
    assert nodes.shape[-1] > 0
    sk, sv, sl = _table(k, v, Q, bs, prototypes)
    assert np.isinf(sl).any() or prototypes == 1 or bs >= prototypes
    out = sparse_attention_summaries(q, k, v, sel, nodes, sk, sv, sl, block_size=bs)
    ref = _bruteforce(q, k, v, sel, nodes, sk, sv, sl, bs)
    np.testing.assert_allclose(out, ref, atol=2e-5, rtol=1e-4)


def test_bruteforce_with_key_padding():
    # Padded batches: row 0 right-padded, row 1 left-padded; padding keys get
    # no weight and the summary table covers the real tokens only.  Real
    # query positions with at least one entry are compared.
    rng = np.random.default_rng(7)
    B, Hq, Hkv, T, D, bs, P = 2, 4, 2, 23, 4, 3, 2
    Q = (T + bs - 1) // bs
    q = rng.standard_normal((B, Hq, T, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    valid = np.zeros((B, T), bool)
    valid[0, :15] = True
    valid[1, 5:] = True
    sel = np.full((B, Hkv, Q, 5), -1, np.int32)
    for b, g, qb in np.ndindex(B, Hkv, Q):
        extra = rng.choice(qb + 1, size=min(qb + 1, 2), replace=False).tolist()
        row = sorted(set(extra) | {qb, max(0, qb - 1)})
        sel[b, g, qb, : len(row)] = row
    nodes = _frontier(sel)
    sk, sv, sl = _table(k, v, Q, bs, P, valid)
    out = sparse_attention_summaries(q, k, v, sel, nodes, sk, sv, sl, block_size=bs, key_valid=valid)
    ref = _bruteforce(q, k, v, sel, nodes, sk, sv, sl, bs, valid)
    for b in range(B):
        for t in range(T):
            if valid[b, t]:
                np.testing.assert_allclose(out[b, t], ref[b, t], atol=2e-5, rtol=1e-4)
    unpadded = sparse_attention_summaries(q, k, v, sel, nodes, *_table(k, v, Q, bs, P), block_size=bs)
    assert np.abs(unpadded[1, 5:] - out[1, 5:]).max() > 1e-2   # the padding changes real rows
