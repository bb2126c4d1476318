"""Seeded synthetic inputs for the sparse-prefill configurations.

Every tensor is drawn from a CPU ``torch.Generator`` (or a numpy
``default_rng`` for block lists) with a recorded seed, in float32, with RoPE
applied in float32 where a configuration asks for it, and only then cast, so
any machine regenerates identical inputs.  Block lists obey the
selected_blocks contract's causal rule; top-k choices use a stable descending
sort (lowest block index wins ties).

Configurations (the names used by bench.py and the tests):
  cfg1  T=4096,   8q/2kv,  d=128, fp32, block mask: top-16 + sink + diagonal
  cfg2  T=32768,  28q/4kv, d=128, bf16+RoPE, block mask ~10% causal density
  cfg5  T=131072, 28q/4kv, d=128, bf16+RoPE, CSR lists, log-normal density
"""
import math

import numpy as np
import torch

BLOCK = 64


def rope(x, theta=1e6):
    """Hugging Face Qwen2 rotary embedding (rotate_half form), positions 0..T-1.

    x: float32 [..., T, D] on any device."""
    T, D = x.shape[-2], x.shape[-1]
    inv_freq = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float32, device=x.device) / D))
    freqs = torch.outer(torch.arange(T, dtype=torch.float32, device=x.device), inv_freq)
    emb = torch.cat([freqs, freqs], dim=-1)
    cos, sin = emb.cos(), emb.sin()
    x1, x2 = x[..., : D // 2], x[..., D // 2:]
    rotated = torch.cat([-x2, x1], dim=-1)
    return x * cos + rotated * sin


def qkv(seed, T, Hq, Hkv, D, dtype, use_rope, B=1, layout="bhtd", device="cpu"):
    """Q [B,Hq,T,D], K/V [B,Hkv,T,D] ~ N(0,1) (float32 draws, then cast).

    layout="bthd" stores Q/K/V as contiguous [B,T,H,D] (Qwen's projection
    layout) and returns the transposed [B,H,T,D] views.  device="cuda" draws
    on the GPU (fast, reproducible on that device, but a different stream of
    numbers than the CPU generator)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    out = []
    for H, rot in ((Hq, use_rope), (Hkv, use_rope), (Hkv, False)):
        x = torch.randn(B, H, T, D, generator=gen, dtype=torch.float32, device=device)
        if rot:
            x = rope(x)
        x = x.to(dtype)
        if layout == "bthd":
            x = x.transpose(1, 2).contiguous().transpose(1, 2)
        out.append(x)
    return tuple(out)


def _stable_topk_desc(scores, k):
    """Indices of the k largest scores, ties to the lowest index."""
    order = np.argsort(-scores, kind="stable")
    return order[:k]


def cfg1_mask(seed=0, T=4096, Hq=8, Hkv=2, top=16):
    """Per KV head: stable top-16 causal key blocks by N(0,1) scores, plus the
    sink block 0 and the diagonal block; expanded to the query heads."""
    qb = (T + BLOCK - 1) // BLOCK
    rng = np.random.default_rng(seed + 1)
    scores = rng.standard_normal((Hkv, qb, qb)).astype(np.float32)
    mask = np.zeros((Hkv, qb, qb), dtype=bool)
    for g in range(Hkv):
        for q in range(qb):
            sel = _stable_topk_desc(scores[g, q, : q + 1], min(top, q + 1))
            mask[g, q, sel] = True
            mask[g, q, 0] = True
            mask[g, q, q] = True
    m = torch.from_numpy(mask)[None].repeat_interleave(Hq // Hkv, dim=1).contiguous()
    return m


def cfg2_mask(seed=0, T=32768, Hq=28, Hkv=4, density=0.10, local=4):
    """Per (KV head, query block): sink {0}, local {q-3..q}, and a stable top-k
    of N(0,1) scores over the remaining causal blocks, with k chosen so each
    row keeps round(density*(q+1)) blocks (never fewer than sink + local).
    Returns (mask [1,Hq,Qb,Qb] bool, realised causal density)."""
    qb = (T + BLOCK - 1) // BLOCK
    rng = np.random.default_rng(seed + 2)
    mask = np.zeros((Hkv, qb, qb), dtype=bool)
    for g in range(Hkv):
        scores = rng.standard_normal((qb, qb)).astype(np.float32)
        for q in range(qb):
            forced = {0} | set(range(max(0, q - local + 1), q + 1))
            want = max(len(forced), int(round(density * (q + 1))))
            mask[g, q, list(forced)] = True
            extra = want - len(forced)
            if extra > 0:
                cand = np.array([j for j in range(1, max(1, q - local + 1))], dtype=np.int64)
                if cand.size:
                    pick = cand[_stable_topk_desc(scores[q, cand], min(extra, cand.size))]
                    mask[g, q, pick] = True
    selected = int(mask.sum())
    causal = Hkv * qb * (qb + 1) // 2
    m = torch.from_numpy(mask)[None].repeat_interleave(Hq // Hkv, dim=1).contiguous()
    return m, selected / causal


def mask_to_selected_blocks(mask_kv):
    """[B, Hkv, Qb, Qb] bool -> padded int32 [B, Hkv, Qb, Kmax] ascending, -1 pad."""
    m = mask_kv.to(torch.bool)
    qb = m.shape[-1]
    counts = m.sum(dim=-1)
    kmax = int(counts.max()) if m.numel() else 0
    ids = torch.arange(qb, dtype=torch.int32).expand_as(m)
    keyed = torch.where(m, ids, torch.full_like(ids, qb))
    packed = keyed.sort(dim=-1).values[..., :kmax]
    return torch.where(packed == qb, torch.full_like(packed, -1), packed).contiguous()


def cfg5_csr(seed=0, T=131072, Hkv=4, median=0.02, sigma=1.0, cap=0.25):
    """CSR block lists with log-normal row densities.

    For row (KV head g, query block q): f ~ LogNormal(ln median, sigma);
    count = min(q+1, max(2, min(round(f*(q+1)), floor(cap*(q+1))))); the row
    holds {0, q} plus a uniform random subset of the other causal blocks,
    sorted ascending.  Returns (indptr int32 [Hkv*Qb+1], indices int32)."""
    qb = (T + BLOCK - 1) // BLOCK
    rng = np.random.default_rng(seed + 5)
    rows = []
    for g in range(Hkv):
        f = rng.lognormal(math.log(median), sigma, size=qb)
        for q in range(qb):
            n = q + 1
            count = min(n, max(2, min(int(round(f[q] * n)), int(math.floor(cap * n)))))
            forced = sorted({0, q})
            extra = count - len(forced)
            if extra > 0 and q > 1:
                others = rng.choice(np.arange(1, q), size=min(extra, q - 1), replace=False)
                row = np.sort(np.concatenate([np.array(forced), others]))
            else:
                row = np.array(forced)
            rows.append(row.astype(np.int32))
    counts = np.array([r.size for r in rows], dtype=np.int64)
    indptr = np.zeros(len(rows) + 1, dtype=np.int64)
    indptr[1:] = np.cumsum(counts)
    indices = np.concatenate(rows).astype(np.int32)
    return torch.from_numpy(indptr.astype(np.int32)), torch.from_numpy(indices)


def attention_flops(selected_head_blocks, D=128):
    """Algorithmic FLOPs: 4*64*64*D per (query head, selected 64-key block)."""
    return 4.0 * BLOCK * BLOCK * D * selected_head_blocks


def cfg3_gate_weights(seed=0, D=128, P=128):
    """Selector gate projections Wq, Wk [D, P] float32, Xavier-uniform, seeded.

    Laid out as FlatGate's per-layer weights (x @ W)."""
    gen = torch.Generator().manual_seed(seed + 3)
    Wq = torch.empty(D, P)
    Wk = torch.empty(D, P)
    torch.nn.init.xavier_uniform_(Wq, generator=gen)
    torch.nn.init.xavier_uniform_(Wk, generator=gen)
    return Wq, Wk


def selector_bytes(T, Hq, Hkv, D, top_k, elem_bytes=2):
    """Compulsory HBM bytes of the selector front end: read Q and K once, write
    the selected indices."""
    nb = (T + BLOCK - 1) // BLOCK
    return (Hq + Hkv) * T * D * elem_bytes + Hkv * nb * top_k * 4


def teacher_flops(T, H, block=BLOCK, D=128):
    """Algorithmic FLOPs of teacher mass: 2*64*64*D per (query head, causal block pair)."""
    qb = (T + block - 1) // block
    return 2.0 * block * block * D * H * qb * (qb + 1) // 2


def tree_route_work(T, Hq, Hkv, D, P=8, proj=128, beam=16, radix=2, k_selected=18, elem_bytes=2):
    """Algorithmic work of each stage of the deployed tree route (prototype
    features -> key tree -> projections -> beam traversal -> packing), one
    layer, batch 1.  Returns {stage: {"bytes": compulsory HBM bytes,
    "flop": arithmetic}}:

    * features: read Q and K once, write the Q and K prototypes
      ([Hkv, nb, P, D] each, model dtype);
    * tree: read the leaf prototypes, write every upper level;
    * project: read the query prototypes and every tree node's prototypes
      (model dtype), write them projected (float32); 2 * D * proj FLOP per
      prototype row;
    * traverse: read the projected tables once, write the leaf ids; per
      query row and tree level the reference scores width * radix candidates
      (scripts/eval_tree_traversal.py:84-113), each P x P prototype pairs of
      2 * proj FLOP;
    * pack: read the int64 leaf ids, write int32 selected_blocks rows.
    """
    nb = (T + BLOCK - 1) // BLOCK
    counts = [nb]
    while counts[-1] > 1:
        counts.append((counts[-1] + radix - 1) // radix)
    nodes = sum(counts)
    width, candidates = 1, 0
    for n in reversed(counts[:-1]):
        candidates += width * radix
        width = min(beam, width * radix, n)
    rows = Hkv * nb
    feat_row = P * D * elem_bytes
    return {
        "features": {"bytes": (Hq + Hkv) * T * D * elem_bytes + 2 * rows * feat_row, "flop": 0},
        "tree": {"bytes": Hkv * nodes * feat_row, "flop": 0},
        "project": {"bytes": Hkv * (nb + nodes) * (feat_row + P * proj * 4),
                    "flop": 2.0 * D * proj * Hkv * (nb + nodes) * P},
        "traverse": {"bytes": Hkv * (nb + nodes) * P * proj * 4 + rows * width * 8,
                     "flop": 2.0 * proj * P * P * candidates * rows,
                     "candidates_per_row": candidates, "width": width},
        "pack": {"bytes": rows * width * 8 + rows * k_selected * 4, "flop": 0},
    }
