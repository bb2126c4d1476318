"""Pins the CPU attention oracle (oracle/attention.py) before it is trusted.

Checks, each chosen so that a plausible oracle mistake fails at least one:
  * the reference's own known answers (tests/test_sparse_attention.py:32-70
    in the reference): all causal blocks == dense masked attention with GQA,
    a pruned block contributes exact zeros, the fp32 score path survives fp16
    overflow;
  * an independent dense closed form over a full [T, T] causal mask;
  * a pure-Python brute force (scalar loops, math.exp, float64) on tiny inputs
    with GQA, a ragged last block, duplicates, unsorted rows, future and
    negative IDs -- catches a wrong head mapping, causal direction, scale or
    output transpose;
  * closed forms: identical keys make attention the plain mean of the
    attended values;
  * the three list layouts (padded, CSR, block mask) agree.
"""
import math

import numpy as np
import pytest
import torch

from oracle.attention import (
    attention_bruteforce,
    dense_causal_attention,
    sparse_attention_csr,
    sparse_attention_index,
    sparse_attention_mask,
)


def _all_causal(qblocks, groups=1, batch=1):
    out = np.full((batch, groups, qblocks, qblocks), -1, dtype=np.int32)
    for q in range(qblocks):
        out[:, :, q, : q + 1] = np.arange(q + 1)
    return out


def test_reference_kat_all_causal_blocks_match_dense_attention():
    # Reference test_sparse_attention.py:32-45 (same seed, shapes, block size 2).
    torch.manual_seed(0)
    query = torch.randn(1, 2, 4, 3)
    key = torch.randn(1, 1, 4, 3)
    value = torch.randn(1, 1, 4, 3)
    out = sparse_attention_index(query.numpy(), key.numpy(), value.numpy(),
                                 _all_causal(2), block_size=2)
    causal = torch.triu(torch.full((4, 4), torch.finfo(torch.float32).min), diagonal=1)
    scores = query @ key.repeat_interleave(2, dim=1).transpose(-1, -2) / math.sqrt(3)
    expected = torch.softmax(scores + causal, dim=-1) @ value.repeat_interleave(2, dim=1)
    assert out.shape == (1, 4, 2, 3)
    np.testing.assert_allclose(out, expected.transpose(1, 2).numpy(), rtol=1.3e-6, atol=1e-5)


def test_reference_kat_pruned_block_cannot_change_output():
    # Reference test_sparse_attention.py:48-59: exact zeros where block 0 is dropped.
    query = np.ones((1, 1, 6, 1), np.float32)
    key = np.ones((1, 1, 6, 1), np.float32)
    value = np.array([7, 7, 0, 0, 0, 0], np.float32).reshape(1, 1, 6, 1)
    selected = np.array([[[[0, -1, -1], [0, 1, -1], [1, 2, -1]]]], np.int32)
    out = sparse_attention_index(query, key, value, selected, block_size=2)
    assert np.array_equal(out[0, 4:, 0], np.zeros_like(out[0, 4:, 0]))
    assert np.all(out[0, :4, 0] > 0)


def test_reference_kat_fp32_scores_survive_fp16_overflow():
    # Reference test_sparse_attention.py:62-70.
    query = np.full((1, 1, 4, 64), 300.0, np.float16)
    key = np.full((1, 1, 4, 64), 300.0, np.float16)
    value = np.arange(4 * 64, dtype=np.float16).reshape(1, 1, 4, 64)
    out = sparse_attention_index(query, key, value, _all_causal(2), block_size=2)
    assert np.isfinite(out).all()


def test_empty_row_raises_like_the_reference():
    q = np.zeros((1, 1, 4, 2), np.float32)
    sel = np.array([[[[0, -1], [-1, -1]]]], np.int32)
    with pytest.raises(ValueError, match="row empty"):
        sparse_attention_index(q, q, q, sel, block_size=2)
    out = sparse_attention_index(q, q, q, sel, block_size=2, empty="zero")
    assert np.array_equal(out[0, 2:], np.zeros_like(out[0, 2:]))


@pytest.mark.parametrize("T", [128, 200])
def test_all_causal_blocks_equal_dense_closed_form(T):
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 6, T, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, T, 64)).astype(np.float32)
    v = rng.standard_normal((1, 2, T, 64)).astype(np.float32)
    qb = (T + 63) // 64
    out = sparse_attention_index(q, k, v, _all_causal(qb, groups=2), block_size=64)
    ref = dense_causal_attention(q, k, v)
    np.testing.assert_allclose(out, ref, atol=2e-5, rtol=1e-4)


def _bruteforce_keys(rows_of, block, T):
    """Key tokens of query t from the row's listed blocks, with multiplicity."""
    def key_sets(b, h, t):
        qb = t // block
        keys = []
        for blk in rows_of(b, h, qb):
            if 0 <= blk <= qb:
                keys.extend(j for j in range(blk * block, min(blk * block + block, T)) if j <= t)
        return keys
    return key_sets


def test_index_oracle_matches_bruteforce_with_messy_rows():
    rng = np.random.default_rng(11)
    B, Hq, Hkv, T, D, bs = 2, 6, 2, 7, 3, 2     # G=3, ragged last block
    qblocks = 4
    q = rng.standard_normal((B, Hq, T, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    idx = np.full((B, Hkv, qblocks, 4), -1, np.int32)
    for b in range(B):
        for g in range(Hkv):
            for qb in range(qblocks):
                row = [qb] + list(rng.integers(-1, qblocks + 1, size=3))  # dups, -1, future
                rng.shuffle(row)
                idx[b, g, qb] = row
    out = sparse_attention_index(q, k, v, idx, block_size=bs)
    ref = attention_bruteforce(
        q, k, v, _bruteforce_keys(lambda b, h, qb: idx[b, h // 3, qb], bs, T))
    np.testing.assert_allclose(out, np.array(ref), atol=1e-5, rtol=1e-5)


def test_per_head_mask_matches_bruteforce():
    rng = np.random.default_rng(5)
    B, Hq, Hkv, T, D, bs = 1, 4, 2, 10, 4, 2
    qblocks = 5
    q = rng.standard_normal((B, Hq, T, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    mask = rng.random((B, Hq, qblocks, qblocks)) < 0.5
    for h in range(Hq):
        for qb in range(qblocks):
            mask[0, h, qb, qb] = True          # keep every row non-empty
    out = sparse_attention_mask(q, k, v, mask, block_size=bs)
    rows = lambda b, h, qb: [j for j in range(qblocks) if mask[b, h, qb, j]]
    ref = attention_bruteforce(q, k, v, _bruteforce_keys(rows, bs, T))
    np.testing.assert_allclose(out, np.array(ref), atol=1e-5, rtol=1e-5)


def test_identical_keys_give_mean_of_attended_values():
    # Closed form: equal scores -> softmax is uniform over the attended keys.
    rng = np.random.default_rng(7)
    T, bs = 12, 4
    q = rng.standard_normal((1, 2, T, 4)).astype(np.float32)
    k = np.ones((1, 1, T, 4), np.float32)
    v = rng.standard_normal((1, 1, T, 4)).astype(np.float32)
    idx = np.array([[[[0, -1], [0, 1], [0, 2]]]], np.int32)
    out = sparse_attention_index(q, k, v, idx, block_size=bs)
    for t in range(T):
        qb = t // bs
        keys = [j for blk in idx[0, 0, qb] if blk >= 0 for j in range(blk * bs, blk * bs + bs) if j <= t]
        np.testing.assert_allclose(out[0, t, 0], v[0, 0, keys].mean(axis=0), atol=1e-6)
        np.testing.assert_allclose(out[0, t, 1], v[0, 0, keys].mean(axis=0), atol=1e-6)


def test_layouts_agree_and_row_order_is_irrelevant():
    rng = np.random.default_rng(9)
    B, Hq, Hkv, T, D, bs = 1, 4, 2, 40, 8, 8
    qblocks = 5
    q = rng.standard_normal((B, Hq, T, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    mask = rng.random((B, Hkv, qblocks, qblocks)) < 0.4
    mask |= np.eye(qblocks, dtype=bool)[None, None]
    rows, idx = [], np.full((B, Hkv, qblocks, qblocks), -1, np.int32)
    for g in range(Hkv):
        for qb in range(qblocks):
            ids = np.nonzero(mask[0, g, qb, : qb + 1])[0]
            rows.append(ids[::-1].astype(np.int32))   # reversed order in CSR
            idx[0, g, qb, : ids.size] = ids
    indptr = np.concatenate([[0], np.cumsum([r.size for r in rows])]).astype(np.int32)
    by_index = sparse_attention_index(q, k, v, idx, block_size=bs)
    by_csr = sparse_attention_csr(q, k, v, indptr, np.concatenate(rows), block_size=bs)
    by_mask = sparse_attention_mask(q, k, v, mask, block_size=bs)
    np.testing.assert_allclose(by_csr, by_index, atol=1e-6)
    np.testing.assert_allclose(by_mask, by_index, atol=1e-6)


def test_key_padding_matches_bruteforce_at_real_positions():
    # Padded batches (sparse/attention.py:225-229 in the reference): padding
    # keys get no weight.  Row 0 right-padded (real tokens 0..4), row 1
    # left-padded (real tokens 3..8); only real query positions are defined.
    rng = np.random.default_rng(5)
    B, Hq, Hkv, T, D, bs = 2, 4, 2, 9, 3, 2
    qblocks = 5
    q = rng.standard_normal((B, Hq, T, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    valid = np.zeros((B, T), bool)
    valid[0, :5] = True
    valid[1, 3:] = True
    idx = np.full((B, Hkv, qblocks, 3), -1, np.int32)
    for b in range(B):
        for g in range(Hkv):
            for qb in range(qblocks):
                row = sorted({0, qb, int(rng.integers(0, qb + 1))})
                idx[b, g, qb, :len(row)] = row
    out = sparse_attention_index(q, k, v, idx, block_size=bs, key_valid=valid)
    listed = _bruteforce_keys(lambda b, h, qb: idx[b, h // 2, qb], bs, T)
    def real_keys(b, h, t):   # padding query positions with no real key are not compared
        keys = [j for j in listed(b, h, t) if valid[b, j]]
        return keys or listed(b, h, t)

    ref = np.array(attention_bruteforce(q, k, v, real_keys))
    for b in range(B):
        for t in range(T):
            if valid[b, t]:
                np.testing.assert_allclose(out[b, t], ref[b, t], atol=1e-5, rtol=1e-5)
    # All keys valid == no key padding.
    np.testing.assert_array_equal(
        sparse_attention_index(q, k, v, idx, block_size=bs, key_valid=np.ones((B, T), bool)),
        sparse_attention_index(q, k, v, idx, block_size=bs))


def test_additive_mask_all_causal_blocks_equal_dense_closed_form():
    # sparse/attention.py:225-229 in the reference adds the mask slice to the
    # scaled scores.  With every causal block listed this is dense attention
    # with the same mask, computed in float64 by an independent closed form;
    # per-head masks (mask head h with query head h) and -inf entries.
    rng = np.random.default_rng(11)
    B, Hq, Hkv, T, D, bs = 2, 4, 2, 10, 5, 4
    q = rng.standard_normal((B, Hq, T, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    for Hm in (1, Hq):
        mask = rng.standard_normal((B, Hm, T, T)).astype(np.float32) * 2
        mask[rng.random(mask.shape) < 0.3] = -np.inf
        diag = np.arange(T)
        mask[:, :, diag, diag] = 0.0        # every row keeps its own key
        out = sparse_attention_index(q, k, v, _all_causal(3, Hkv, B), block_size=bs,
                                     add_mask=mask)
        ref = dense_causal_attention(q, k, v, add_mask=mask)
        np.testing.assert_allclose(out, ref, atol=2e-6, rtol=2e-5)


def test_additive_mask_matches_bruteforce_with_messy_rows():
    # Finite biases on listed keys, GQA, a ragged last block, unsorted rows
    # with a duplicate and a future block: the mask is indexed by the listed
    # key (not its position in the row) and by the query's own head.
    rng = np.random.default_rng(12)
    B, Hq, Hkv, T, D, bs = 1, 4, 2, 7, 3, 2
    q = rng.standard_normal((B, Hq, T, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    mask = rng.standard_normal((B, Hq, T, T)).astype(np.float32)
    idx = np.array([[[[0, -1, -1], [1, 0, 1], [2, 3, 0], [3, 1, -1]],
                     [[0, 1, -1], [0, -1, -1], [1, 2, -1], [2, 3, 0]]]], np.int32)
    out = sparse_attention_index(q, k, v, idx, block_size=bs, add_mask=mask)
    ref = attention_bruteforce(q, k, v, _bruteforce_keys(lambda b, h, qb: idx[b, h // 2, qb], bs, T),
                               bias=lambda b, h, t, j: float(mask[b, h, t, j]))
    np.testing.assert_allclose(out, np.array(ref), atol=1e-5, rtol=1e-5)


def test_additive_padding_mask_equals_key_padding():
    # A 0 / finfo.min mask that is causal key padding gives the key-padding
    # path's result at every real query position.
    rng = np.random.default_rng(13)
    B, Hq, Hkv, T, D, bs = 2, 2, 1, 9, 4, 4
    q = rng.standard_normal((B, Hq, T, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
    valid = np.zeros((B, T), bool)
    valid[0, :6] = True
    valid[1, 2:] = True
    allowed = np.tril(np.ones((T, T), bool))[None] & valid[:, None, :]
    mask = np.where(allowed, 0.0, np.finfo(np.float32).min).astype(np.float32)[:, None]
    idx = _all_causal(3, Hkv, B)
    by_mask = sparse_attention_index(q, k, v, idx, block_size=bs, add_mask=mask)
    by_valid = sparse_attention_index(q, k, v, idx, block_size=bs, key_valid=valid)
    np.testing.assert_allclose(by_mask[valid], by_valid[valid], atol=1e-6, rtol=1e-6)


def test_packed_sequences_equal_each_sequence_alone():
    # A block-diagonal mask over packed sequences: every sequence's output
    # equals its attention computed alone (block-aligned starts, so the
    # sequence's own blocks are a causal prefix of its own token range).
    rng = np.random.default_rng(14)
    Hq, Hkv, D, bs = 2, 1, 4, 4
    lengths = [8, 5, 7]
    starts = np.cumsum([0] + [8, 8])
    T = int(starts[-1] + lengths[-1])
    q = rng.standard_normal((1, Hq, T, D)).astype(np.float32)
    k = rng.standard_normal((1, Hkv, T, D)).astype(np.float32)
    v = rng.standard_normal((1, Hkv, T, D)).astype(np.float32)
    seg = np.full(T, -1)
    for i, (s0, n) in enumerate(zip(starts, lengths)):
        seg[s0:s0 + n] = i
    same = (seg[:, None] == seg[None, :]) & (seg[:, None] >= 0)
    mask = np.where(same, 0.0, -np.inf).astype(np.float32)[None, None]
    out = sparse_attention_index(q, k, v, _all_causal(-(-T // bs)), block_size=bs, add_mask=mask)
    for s0, n in zip(starts, lengths):
        alone = dense_causal_attention(q[:, :, s0:s0 + n], k[:, :, s0:s0 + n], v[:, :, s0:s0 + n])
        np.testing.assert_allclose(out[:, s0:s0 + n], alone, atol=2e-6, rtol=2e-5)
