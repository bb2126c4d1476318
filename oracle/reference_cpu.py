"""Torch CPU restatements of the reference's own CPU paths -- TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's cpu_baseline legs use this module: as the CPU
baseline the benchmark times (the reference path restated with torch ops on
the host cores, in float32) and, in float64, as the reference-order
comparison of the selector robustness test.  Nothing in the shipped package
imports it.

  flat_select      the flat selector of the reference's evaluation route, in
                   the reference's op order: _group_avg_tokens (a mean over
                   the G query heads of each KV group per token,
                   teacher/chunked_extract.py:75-80), 64-token block means
                   (prototype 0 of _proto_pool_seq, :46-47) of the grouped
                   queries and of the keys, the per-dim block max of the keys
                   (the cfg3 max summary, which the reference does not have),
                   FlatGate._layer_scores (selector/gate.py:47-78: einsum
                   projections, running max over key prototypes of the max
                   over query prototypes), the 1/sqrt(p) of FlatGate.forward
                   (:101), the causal masked_fill with finfo.min
                   (selector/recall.py:26-29) and the stable descending
                   argsort of selector/baselines.py:59-62 (ties to the lower
                   block index); rows written ascending with -1 padding, the
                   selected_blocks layout.
  chunked_pool     teacher/chunked_extract.py:91-130: per head chunk and query
                   block the causal score strip, -inf above the diagonal, a
                   float32 row softmax, 64-key sums, then the sum over the
                   block's rows.  K is read at KV resolution (query head h
                   reads KV head h // G, what _repeat_kv expands, :83-88);
                   scores are formed in float32 from the upcast inputs.
  teacher_targets  selector/targets.py:104-121 (group mean, causal mask, row
                   normalisation with eps) plus the top-k target blocks of
                   selector/loss.py:34-46 (target.topk).
  group_mass       the first half of teacher_targets alone (the mass that
                   load_teacher keeps with defer_normalization).
"""
import math

import torch

BLOCK = 64


def _stable_topk_rows(scores, top_k):
    """scores [R, Qb, Kb] (causally masked) -> int32 [R, Qb, top_k]: the stable
    descending argsort of each row's causal entries, first top_k, ascending,
    -1 padding (selector/baselines.py:59-62)."""
    R, Qb, Kb = scores.shape
    order = torch.argsort(scores, dim=-1, descending=True, stable=True)[..., :top_k]
    qpos = torch.arange(Qb)[None, :, None]
    rank = torch.arange(top_k)[None, None, :]
    order = torch.where(rank <= qpos, order, torch.full_like(order, Kb))  # rows with q+1 < top_k
    order = torch.sort(order, dim=-1).values
    return torch.where(order < Kb, order, torch.full_like(order, -1)).to(torch.int32)


@torch.no_grad()
def flat_select(q, k, Wq, Wk, top_k=32, dtype=torch.float32, return_scores=False):
    """q [1, Hq, T, D], k [1, Hkv, T, D] (T a multiple of 64), Wq/Wk [D, P].

    Returns selected int32 [1, 1, Hkv, nb, top_k] (and the masked scores
    [Hkv, nb, nb] when return_scores)."""
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    if B != 1 or T % BLOCK:
        raise ValueError("flat_select restates the batch-1, whole-block cfg3 path")
    rep, nb = Hq // Hkv, T // BLOCK
    qf = q.to(dtype).view(Hkv, rep, T, D).mean(dim=1)              # _group_avg_tokens
    q_feat = qf.view(Hkv, nb, BLOCK, D).mean(dim=2)[:, :, None]   # [G, nb, 1, D]
    kf = k.to(dtype)[0].view(Hkv, nb, BLOCK, D)
    k_feat = torch.stack([kf.mean(dim=2), kf.amax(dim=2)], dim=2)  # [G, nb, 2, D]
    Wq, Wk = Wq.to(dtype), Wk.to(dtype)
    qp = torch.einsum("gqid,dp->gqip", q_feat, Wq)
    kp = torch.einsum("gkjd,dp->gkjp", k_feat, Wk)
    best = None
    for j in range(kp.shape[2]):
        s = torch.einsum("gqip,gkp->gqik", qp, kp[:, :, j, :]).max(dim=2).values
        best = s if best is None else torch.where(s > best, s, best)
    scores = best / math.sqrt(Wq.shape[1])
    cmask = torch.arange(nb)[None, :] <= torch.arange(nb)[:, None]
    scores = scores.masked_fill(~cmask[None], torch.finfo(scores.dtype).min)
    sel = _stable_topk_rows(scores, min(top_k, nb))[None, None]
    return (sel, scores) if return_scores else sel


@torch.no_grad()
def chunked_pool(query, key, scaling, block=BLOCK, head_chunk=2, heads=None):
    """query [b, H, T, d], key [b, Hkv, T, d] -> float32 mass [b, H, qb, qb]
    (rows of heads outside ``heads`` stay zero)."""
    b, H, T, d = query.shape
    G = H // key.shape[1]
    qb = (T + block - 1) // block
    q32, k32 = query.float(), key.float()
    pooled = torch.zeros((b, H, qb, qb), dtype=torch.float32)
    todo = list(range(H)) if heads is None else list(heads)
    for c in range(0, len(todo), head_chunk):
        hs = todo[c:c + head_chunk]
        kidx = torch.tensor([h // G for h in hs])
        for I in range(qb):
            r0, r1 = I * block, min((I + 1) * block, T)
            end = r1
            kb_up = (end + block - 1) // block
            s = torch.matmul(q32[:, hs, r0:r1], k32[:, kidx, :end].transpose(-1, -2)) * scaling
            g = torch.arange(r0, r1)[:, None]
            j = torch.arange(end)[None, :]
            s = s.masked_fill((j > g)[None, None], float("-inf"))
            p = torch.softmax(s, dim=-1)
            p = torch.nn.functional.pad(p, (0, kb_up * block - end))
            p = p.view(b, len(hs), r1 - r0, kb_up, block).sum(dim=-1)
            pooled[:, hs, I, :kb_up] = p.sum(dim=2)
    return pooled


@torch.no_grad()
def group_mass(mass, num_kv_heads):
    """mass [b, H, qb, kb] -> the KV-group mean with the causal mask
    [b, G, qb, kb] (selector/targets.py:104-108, the mass load_teacher keeps
    with defer_normalization)."""
    b, H, qb, kb = mass.shape
    m = mass.view(b, num_kv_heads, H // num_kv_heads, qb, kb).mean(dim=2)
    cmask = torch.arange(kb)[None, :] <= torch.arange(qb)[:, None]
    return m * cmask


@torch.no_grad()
def teacher_targets(mass, num_kv_heads, eps=1e-9, k=8):
    """mass [b, H, qb, kb] -> (target [b, G, qb, kb], row_mass [b, G, qb],
    topk int64 [b, G, qb, k])."""
    b, H, qb, kb = mass.shape
    m = mass.view(b, num_kv_heads, H // num_kv_heads, qb, kb).mean(dim=2)
    cmask = torch.arange(kb)[None, :] <= torch.arange(qb)[:, None]
    m = m * cmask
    row = m.sum(dim=-1, keepdim=True)
    target = m / row.clamp_min(eps)
    return target, row.squeeze(-1), target.topk(k, dim=-1).indices
