"""CPU oracle for block-sparse causal GQA prefill attention.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this file;
only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
as the checker of the HIP kernels.

Restates the reference's PyTorch oracle, sparse/attention.py:186-274, in
numpy float32:
  for each query block qb, batch b and KV head g (sparse/attention.py:186-191)
    ids  = selected[b, g, qb][selected >= 0]            (:192-199; empty -> ValueError)
    keys = ids * block + arange(block), keeping keys < T (:204-207)
    s    = (q_blk @ k_sel^T) / sqrt(D) in float32       (:217-219)
    s[key > query] = finfo.min                          (:223-224)
    out  = softmax(s) @ v_sel                           (:266-269)
and returns [B, T, Hq, D] (:274).

Deliberate, documented choices where the reference has no single answer:
  * block IDs above the query block are dropped.  In the reference oracle such
    a block is fully masked and adds exactly zero weight whenever the row has
    any causal key; for a row made only of future blocks the reference's
    backends disagree (its oracle averages V uniformly, its Triton kernel
    yields NaN).  Here such a row counts as empty;
  * duplicated IDs are kept and attended twice, as the reference oracle does;
  * ``scale`` defaults to 1/sqrt(D) (the reference divides by math.sqrt(D));
  * ``qblocks_subset`` computes only the listed query blocks (the others stay
    zero), so full-size configurations can be spot-checked row by row.

``sparse_attention_index(add_mask=...)`` restates the additive 4-D mask of
sparse/attention.py:225-229: the mask slice at the row's queries and listed
keys is added to the scores after the causal fill.

``sparse_attention_summaries`` restates the residual-summary branch
(sparse/attention.py:226-265): the row's exact keys plus, for each listed tree
node and prototype with a non-zero count, the summary key with score
q . k / sqrt(D) + log(count) and the summary value, in one softmax.

Pinned by tests/test_oracle_attention.py against the reference's own known
answers (tests/test_sparse_attention.py:32-87 there), an independent dense
closed form, a pure-Python brute force and structural invariants; the
additive mask by the dense closed form with the same mask, the brute force
with per-key biases, the key-padding path, and packed sequences that must
equal each sequence attended alone.
"""
import math

import numpy as np

F32_MIN = np.finfo(np.float32).min


def _softmax_rows(s):
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    return p / p.sum(axis=-1, keepdims=True)


def _attend_group(qblk, keys, vals, q_pos, key_idx, scale, key_ok=None, bias=None):
    """qblk [H, n, D], keys/vals [m, D] -> [H, n, D] (float32).  key_ok [m]:
    key padding, scored finfo.min like the causal fill.  bias [H or 1, n, m]:
    the additive mask slice, added after the causal fill
    (sparse/attention.py:223-229); finfo.min + finfo.min overflows to -inf in
    float32 there too.  A row whose every score is -inf is NaN, as the
    reference's softmax makes it."""
    s = np.matmul(qblk, keys.T) * np.float32(scale) if scale is not None else \
        np.matmul(qblk, keys.T) / np.float32(math.sqrt(qblk.shape[-1]))
    causal = key_idx[None, :] <= q_pos[:, None]
    if key_ok is not None:
        causal = causal & key_ok[None, :]
    s = np.where(causal[None], s, F32_MIN)
    if bias is not None:
        with np.errstate(over="ignore", invalid="ignore"):
            s = (s + bias.astype(np.float32)).astype(np.float32)
    with np.errstate(invalid="ignore"):
        return np.matmul(_softmax_rows(s), vals).astype(np.float32)


def _sparse_attention(q, k, v, blocks_for, block_size, scale, empty, qblocks_subset=None, key_valid=None,
                      add_mask=None):
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    if Hq % Hkv:
        raise ValueError("query heads must be divisible by KV heads")
    G = Hq // Hkv
    qblocks = (T + block_size - 1) // block_size
    out = np.zeros((B, Hq, T, D), dtype=np.float32)
    offs = np.arange(block_size)
    for qb in (range(qblocks) if qblocks_subset is None else qblocks_subset):
        q0, q1 = qb * block_size, min((qb + 1) * block_size, T)
        q_pos = np.arange(q0, q1)
        for b in range(B):
            for g in range(Hkv):
                per_head = blocks_for(b, g, qb)
                if isinstance(per_head, list):  # one list per query head
                    work = [(slice(g * G + h, g * G + h + 1), per_head[h]) for h in range(G)]
                else:  # one list shared by the KV head's G query heads
                    work = [(slice(g * G, (g + 1) * G), per_head)]
                for heads, ids in work:
                    ids = np.asarray(ids, dtype=np.int64)
                    ids = ids[(ids >= 0) & (ids <= qb)]
                    if ids.size == 0:
                        if empty == "zero":
                            continue
                        raise ValueError(
                            "selected_blocks leaves an attention row empty at "
                            f"batch={b}, kv_head={g}, query_block={qb}")
                    key_idx = (ids[:, None] * block_size + offs[None, :]).reshape(-1)
                    key_idx = key_idx[key_idx < T]
                    key_ok = None if key_valid is None else np.asarray(key_valid[b], dtype=bool)[key_idx]
                    bias = None
                    if add_mask is not None:
                        mh = heads if add_mask.shape[1] > 1 else slice(0, 1)
                        bias = add_mask[b, mh, q0:q1][..., key_idx]
                    out[b, heads, q0:q1] = _attend_group(
                        q[b, heads, q0:q1], k[b, g, key_idx], v[b, g, key_idx],
                        q_pos, key_idx, scale, key_ok, bias)
    return out.transpose(0, 2, 1, 3).copy()


def sparse_attention_index(q, k, v, idx, block_size=64, scale=None, empty="raise",
                           qblocks_subset=None, key_valid=None, add_mask=None):
    """Padded direct-index lists ``idx [B, Hkv, Qb, K]`` -> ``[B, T, Hq, D]``.

    key_valid: optional bool ``[B, T]`` key padding; padding keys get the
    finfo.min score of the reference's additive decoder mask
    (sparse/attention.py:225-229).  Rows at padding query positions whose
    listed causal keys are all padding are then a uniform average (the
    reference's result too); callers compare real positions only.

    add_mask: optional additive mask ``[B, 1 or Hq, >=T, >=T]`` (float; -inf
    allowed), whose slice at the row's queries and listed keys is added to
    the scores after the causal fill, as sparse/attention.py:225-229 adds
    ``attention_mask[b, :, q0:q1].index_select(-1, keys)``.  Mask head h goes
    with query head h."""
    idx = np.asarray(idx)
    if add_mask is not None:
        add_mask = np.asarray(add_mask, dtype=np.float32)
    return _sparse_attention(q, k, v, lambda b, g, qb: idx[b, g, qb], block_size, scale, empty,
                             qblocks_subset, key_valid, add_mask)


def sparse_attention_csr(q, k, v, indptr, indices, block_size=64, scale=None, empty="raise",
                         qblocks_subset=None):
    """CSR lists, row ``(b*Hkv + g)*Qb + qb`` -> ``[B, T, Hq, D]``."""
    indptr = np.asarray(indptr)
    indices = np.asarray(indices)
    T = np.asarray(q).shape[2]
    Hkv = np.asarray(k).shape[1]
    qblocks = (T + block_size - 1) // block_size

    def blocks_for(b, g, qb):
        r = (b * Hkv + g) * qblocks + qb
        return indices[indptr[r]:indptr[r + 1]]

    return _sparse_attention(q, k, v, blocks_for, block_size, scale, empty, qblocks_subset)


def sparse_attention_mask(q, k, v, mask, block_size=64, scale=None, empty="raise",
                          qblocks_subset=None):
    """Boolean block mask ``[B, Hm, Qb, >=Qb]`` with Hm == Hq or Hkv."""
    mask = np.asarray(mask).astype(bool)
    Hq = np.asarray(q).shape[1]
    Hkv = np.asarray(k).shape[1]
    G = Hq // Hkv
    Hm = mask.shape[1]

    def blocks_for(b, g, qb):
        if Hm == Hq and G > 1:
            rows = [np.nonzero(mask[b, g * G + h, qb, :qb + 1])[0] for h in range(G)]
            if all(np.array_equal(rows[0], r) for r in rows[1:]):
                return rows[0]
            return rows
        return np.nonzero(mask[b, g, qb, :qb + 1])[0]

    return _sparse_attention(q, k, v, blocks_for, block_size, scale, empty, qblocks_subset)


def dense_causal_attention(q, k, v, scale=None, add_mask=None):
    """Closed form: full [T, T] causal softmax attention, GQA by head repetition.

    Independent of the block gather above; used to pin it (all causal blocks
    selected must reproduce this).  add_mask ``[B, 1 or Hq, T, T]`` is added
    to the scaled scores (float64; -inf masks)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, T, D = q.shape
    G = Hq // k.shape[1]
    kr = np.repeat(k, G, axis=1)
    vr = np.repeat(v, G, axis=1)
    s = np.matmul(q, kr.transpose(0, 1, 3, 2)) * (scale if scale is not None else 1.0 / math.sqrt(D))
    future = np.triu(np.ones((T, T), dtype=bool), k=1)
    s = np.where(future[None, None], -np.inf, s)
    if add_mask is not None:
        s = s + np.asarray(add_mask, dtype=np.float64)[:, :, :T, :T]
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.matmul(p, vr).transpose(0, 2, 1, 3)


def attention_bruteforce(q, k, v, key_sets, scale=None, bias=None):
    """Pure-Python loops (math.exp, no numpy reductions) for tiny inputs.

    key_sets(b, hq, t) -> iterable of key token indices attended by query t of
    query head hq; bias(b, hq, t, j) -> finite number added to key j's score.
    Returns nested lists [B][T][Hq][D]."""
    q = np.asarray(q, dtype=np.float64).tolist()
    k = np.asarray(k, dtype=np.float64).tolist()
    v = np.asarray(v, dtype=np.float64).tolist()
    B, Hq, T, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    G = Hq // len(k[0])
    sc = scale if scale is not None else 1.0 / math.sqrt(D)
    out = [[[[0.0] * D for _ in range(Hq)] for _ in range(T)] for _ in range(B)]
    for b in range(B):
        for h in range(Hq):
            g = h // G
            for t in range(T):
                keys = list(key_sets(b, h, t))
                scores = [sum(q[b][h][t][d] * k[b][g][j][d] for d in range(D)) * sc
                          + (bias(b, h, t, j) if bias is not None else 0.0) for j in keys]
                mx = max(scores)
                w = [math.exp(s - mx) for s in scores]
                z = sum(w)
                for d in range(D):
                    out[b][t][h][d] = sum(wi * v[b][g][j][d] for wi, j in zip(w, keys)) / z
    return out


def sparse_attention_summaries(q, k, v, idx, nodes, sum_keys, sum_values, sum_log_counts,
                               block_size=64, scale=None, qblocks_subset=None, key_valid=None):
    """Padded lists ``idx [B,Hkv,Qb,K]`` plus summary rows ``nodes [B,Hkv,Qb,S]``
    over a table ``sum_keys/sum_values [B,Hkv,N,P,D]``, ``sum_log_counts
    [B,N,P]`` (natural log, -inf for empty prototypes) -> ``[B,T,Hq,D]``.
    key_valid: optional bool ``[B, T]`` key padding of the exact keys (the
    table is then built over the real tokens only)."""
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    idx, nodes = np.asarray(idx), np.asarray(nodes)
    sk = np.asarray(sum_keys, dtype=np.float32)
    sv = np.asarray(sum_values, dtype=np.float32)
    sl = np.asarray(sum_log_counts, dtype=np.float32)
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    N = sk.shape[2]
    def scaled(x):  # the reference divides by sqrt(D) (sparse/attention.py:217-219, 253-256)
        return x * np.float32(scale) if scale is not None else x / np.float32(math.sqrt(D))

    qblocks = (T + block_size - 1) // block_size
    out = np.zeros((B, Hq, T, D), dtype=np.float32)
    offs = np.arange(block_size)
    for qb in (range(qblocks) if qblocks_subset is None else qblocks_subset):
        q0, q1 = qb * block_size, min((qb + 1) * block_size, T)
        q_pos = np.arange(q0, q1)
        for b in range(B):
            for g in range(Hkv):
                ids = np.asarray(idx[b, g, qb], dtype=np.int64)
                ids = ids[(ids >= 0) & (ids <= qb)]
                if ids.size == 0:
                    raise ValueError(
                        "selected_blocks leaves an attention row empty at "
                        f"batch={b}, kv_head={g}, query_block={qb}")
                key_idx = (ids[:, None] * block_size + offs[None, :]).reshape(-1)
                key_idx = key_idx[key_idx < T]
                heads = slice(g * G, (g + 1) * G)
                qh = q[b, heads, q0:q1]
                s = scaled(np.matmul(qh, k[b, g, key_idx].T))
                ok = key_idx[None, :] <= q_pos[:, None]
                if key_valid is not None:
                    ok = ok & np.asarray(key_valid[b], dtype=bool)[key_idx][None, :]
                s = np.where(ok[None], s, F32_MIN)
                vals = v[b, g, key_idx]
                row = np.asarray(nodes[b, g, qb], dtype=np.int64)
                row = row[(row >= 0) & (row < N)]
                if row.size:
                    keys_s = sk[b, g, row].reshape(-1, D)
                    vals_s = sv[b, g, row].reshape(-1, D)
                    bias = sl[b, row].reshape(-1)
                    keep = np.isfinite(bias)
                    if keep.any():
                        ss = scaled(np.matmul(qh, keys_s[keep].T)) + bias[keep][None, None, :]
                        s = np.concatenate([s, ss.astype(np.float32)], axis=-1)
                        vals = np.concatenate([vals, vals_s[keep]], axis=0)
                out[b, heads, q0:q1] = np.matmul(_softmax_rows(s), vals).astype(np.float32)
    return out.transpose(0, 2, 1, 3).copy()
