"""CPU oracle for teacher target extraction -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, as the checker of the HIP teacher kernels.

Restatements (numpy, float64 unless noted):
  block_mass     chunked_pool (teacher/chunked_extract.py:91-131): per (batch,
                 head, query block I) the causal score strip q_I k[:end]^T *
                 scale, -inf above the diagonal, a row softmax, key-block sums,
                 then the sum over the block's query rows.  Scores are formed
                 in float64 from the inputs as given (the reference rounds
                 QK^T to the model dtype first, :119); query head h reads KV
                 head h // (H / Hkv) (the _repeat_kv expansion, :83-88).
  pool_attention teacher/pool.py:3-21 (block sums of a full attention map).
  rollup         teacher/pool.py:23-39 (2x2 parent sums until a dim is odd).
  check_causal   teacher/validate.py:3-15.
  targets        selector/targets.py:104-121 (mean over each KV group's query
                 heads, causal mask, row normalisation with eps) plus the
                 top-k target blocks (selector/loss.py:34-46) ordered by
                 target descending, ties to the lower block index, -1 padding.

Pinned by tests/test_oracle_teacher.py: block_mass equals pool_attention of a
dense causal softmax (an independent full-matrix computation), rows of mass
sum to the number of real query rows, the upper triangle is exactly zero,
rollup preserves totals, targets rows sum to one.
"""
import math

import numpy as np


def block_mass(q, k, block=64, scale=None, rows=None):
    """q [B,H,T,D], k [B,Hkv,T,D] -> mass [B,H,Qb,Qb] (float64).

    rows: optional iterable of (b, h, I) to compute; the rest stay zero."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    B, H, T, D = q.shape
    G = H // k.shape[1]
    qb = (T + block - 1) // block
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    mass = np.zeros((B, H, qb, qb), dtype=np.float64)
    todo = rows if rows is not None else [(b, h, I) for b in range(B) for h in range(H) for I in range(qb)]
    for b, h, I in todo:
        r0, r1 = I * block, min((I + 1) * block, T)
        s = q[b, h, r0:r1] @ k[b, h // G, :r1].T * sc
        gi = np.arange(r0, r1)[:, None]
        j = np.arange(r1)[None, :]
        s = np.where(j > gi, -np.inf, s)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        kb_up = (r1 + block - 1) // block
        p = np.pad(p, ((0, 0), (0, kb_up * block - r1)))
        mass[b, h, I, :kb_up] = p.reshape(r1 - r0, kb_up, block).sum(axis=(0, 2))
    return mass


def dense_causal_softmax(q, k, scale=None):
    """Full [B,H,T,T] causal attention probabilities (GQA by head repetition)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    B, H, T, D = q.shape
    G = H // k.shape[1]
    kr = np.repeat(k, G, axis=1)
    s = q @ kr.transpose(0, 1, 3, 2) * (1.0 / math.sqrt(D) if scale is None else scale)
    s = np.where(np.triu(np.ones((T, T), bool), k=1)[None, None], -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    return p / p.sum(axis=-1, keepdims=True)


def pool_attention(attn, block):
    """[b,h,q,k] -> [b,h,qb,kb] block sums (teacher/pool.py:3-21)."""
    b, h, ql, kl = attn.shape
    qb, kb = (ql + block - 1) // block, (kl + block - 1) // block
    padded = np.pad(attn, ((0, 0), (0, 0), (0, qb * block - ql), (0, kb * block - kl)))
    return padded.reshape(b, h, qb, block, kb, block).sum(axis=(3, 5))


def rollup(pooled):
    """Leaf-first list of levels, each the 2x2 sum of the previous (teacher/pool.py:23-39)."""
    levels = [pooled]
    cur = pooled
    while cur.shape[-1] >= 2 and cur.shape[-2] >= 2:
        b, h, qb, kb = cur.shape
        if qb % 2 or kb % 2:
            break
        cur = cur.reshape(b, h, qb // 2, 2, kb // 2, 2).sum(axis=(3, 5))
        levels.append(cur)
    return levels


def check_causal(pooled, tolerance=1e-6):
    """(ok, first (i, j) with leakage above the diagonal) (teacher/validate.py:3-15)."""
    _, _, qb, kb = pooled.shape
    for i in range(qb):
        for j in range(i + 1, kb):
            if np.abs(pooled[:, :, i, j]).max() > tolerance:
                return False, (i, j)
    return True, None


def targets(mass, num_kv_heads, eps=1e-9, k=8):
    """mass [B,H,Qb,Kb] -> (target [B,G,Qb,Kb], row_mass [B,G,Qb], topk int32 [B,G,Qb,k])."""
    mass = np.asarray(mass, dtype=np.float64)
    B, H, Qb, Kb = mass.shape
    G = num_kv_heads
    m = mass.reshape(B, G, H // G, Qb, Kb).mean(axis=2)
    causal = np.arange(Kb)[None, :] <= np.arange(Qb)[:, None]
    m = m * causal[None, None]
    row = m.sum(axis=-1, keepdims=True)
    target = m / np.maximum(row, eps)
    top = np.full((B, G, Qb, k), -1, np.int32)
    for b in range(B):
        for g in range(G):
            for i in range(Qb):
                n = min(i + 1, Kb)
                order = np.argsort(-target[b, g, i, :n], kind="stable")[:k]
                top[b, g, i, : order.size] = order
    return target, row[..., 0], top
