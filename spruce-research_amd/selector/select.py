"""Flat selector front end on gfx950: pool -> project -> MaxSim score -> causal top-k.

The flat route of the reference's selector (scripts/eval_gate.py:70-72):
FlatGate scoring (selector/gate.py:29-101) over pooled block features
(teacher/chunked_extract.py:27-80), the causal mask and top-k of
selector/recall.py:26-35 with the stable lowest-index tie rule of
selector/baselines.py:59-62, producing rows in the selected_blocks layout
(interfaces/selected_blocks_spec.md).  Every step is one HIP kernel behind the
C ABI; the float results are bit-reproducible (fixed IEEE operation order), so
the selected indices are exactly those of the CPU restatement.

Shapes follow the reference: query ``[B,Hq,T,D]``, key ``[B,Hkv,T,D]`` (any
strides with a contiguous last dim), gate weights ``[D, P]`` float32 (one
layer of FlatGate's ``[L, d, p]``).
"""
import ctypes
import math

import torch

import spruce_hip

BLOCK = 64


def _cuda(t, name):
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (HIP selector)")


def pool_blocks(query=None, key=None):
    """Per-64-token-block summaries.

    query ``[B,Hq,T,D]`` -> ``q_mean [B,Hkv,nb,D]`` float32: query heads averaged
    within each KV group per token, then the block mean (needs ``key`` for Hkv
    or pass ``num_kv_heads`` via key's shape).  key ``[B,Hkv,T,D]`` ->
    ``k_sum [B,Hkv,nb,2,D]`` float32: block mean and per-dim block max.
    """
    if query is None and key is None:
        raise ValueError("pool_blocks needs query and/or key")
    ref = key if key is not None else query
    _cuda(ref, "key" if key is not None else "query")
    if key is None:
        raise ValueError("pool_blocks needs key to know the KV head count")
    B, Hkv, T, D = key.shape
    Hq = query.shape[1] if query is not None else Hkv
    if query is not None:
        _cuda(query, "query")
        if query.shape[0] != B or query.shape[2:] != key.shape[2:] or Hq % Hkv:
            raise ValueError("query must be [B, Hq, T, D] with Hq a multiple of key's KV heads")
        if query.dtype != key.dtype:
            raise ValueError("query and key must share a dtype")
    if D % 8:
        raise ValueError(f"head_dim must be a multiple of 8, got {D}")
    nb = (T + BLOCK - 1) // BLOCK
    q_mean = torch.empty((B, Hkv, nb, D), device=key.device, dtype=torch.float32) if query is not None else None
    k_sum = torch.empty((B, Hkv, nb, 2, D), device=key.device, dtype=torch.float32)
    with torch.cuda.device(key.device):
        rc = spruce_hip.lib().spruce_selector_pool(
            spruce_hip.ptr(query), spruce_hip.strides(query) if query is not None else None,
            spruce_hip.ptr(key), spruce_hip.strides(key),
            B, Hq, Hkv, T, D, spruce_hip.dtype_code(key),
            spruce_hip.ptr(q_mean), spruce_hip.ptr(k_sum), spruce_hip.stream_of(key))
    spruce_hip.check(rc, "spruce_selector_pool")
    return q_mean, k_sum


def pool_project_applies(query, key, Wq, Wk):
    """True when ``pool_project`` covers the shapes: head_dim and projection
    dim 128 (one ``[128, 128]`` float32 weight per side), bf16 or fp16 query
    and key of one dtype, at most 8 query heads per KV head, each (batch, KV
    group) slice of q and k within 2^31 bytes."""
    if query is None or key is None or query.dim() != 4 or key.dim() != 4:
        return False
    if Wq.dim() != 2 or Wq.shape != (128, 128) or Wk.shape != (128, 128):
        return False
    if Wq.dtype != torch.float32 or Wk.dtype != torch.float32:
        return False
    if query.dtype != key.dtype or query.dtype not in (torch.bfloat16, torch.float16):
        return False
    B, Hq, T, D = query.shape
    Hkv = key.shape[1]
    if D != 128 or key.shape[0] != B or key.shape[2:] != query.shape[2:] or Hq % Hkv or Hq // Hkv > 8:
        return False
    qs, ks = query.stride(), key.stride()
    if qs[3] != 1 or ks[3] != 1 or min(qs[1], qs[2], ks[2]) < 0:
        return False
    G = Hq // Hkv
    return ((T - 1) * qs[2] + (G - 1) * qs[1] + D) * 2 < 2 ** 31 and ((T - 1) * ks[2] + D) * 2 < 2 ** 31


def pool_project(query, key, Wq, Wk):
    """``project_pair(*pool_blocks(query, key), ...)`` in one launch, for the
    shapes of ``pool_project_applies``: returns ``qp [B,Hkv,nb,P]`` and
    ``kp [B,Hkv,nb,2,P]`` float32, the same values (same operation order)
    without the pooled summaries or a second launch."""
    _cuda(query, "query")
    _cuda(key, "key")
    if not pool_project_applies(query, key, Wq, Wk):
        raise ValueError("pool_project needs head_dim 128, [128, 128] float32 weights, bf16/fp16 inputs and "
                         "at most 8 query heads per KV head")
    B, Hq, T, D = query.shape
    Hkv = key.shape[1]
    P = Wq.shape[1]
    nb = (T + BLOCK - 1) // BLOCK
    Wq = Wq.to(query.device).contiguous()
    Wk = Wk.to(query.device).contiguous()
    qp = torch.empty((B, Hkv, nb, P), device=query.device, dtype=torch.float32)
    kp = torch.empty((B, Hkv, nb, 2, P), device=query.device, dtype=torch.float32)
    with torch.cuda.device(query.device):
        rc = spruce_hip.lib().spruce_selector_pool_project(
            spruce_hip.ptr(query), spruce_hip.strides(query), spruce_hip.ptr(key), spruce_hip.strides(key),
            B, Hq, Hkv, T, D, spruce_hip.dtype_code(query), spruce_hip.ptr(Wq), spruce_hip.ptr(Wk), P,
            spruce_hip.ptr(qp), spruce_hip.ptr(kp), spruce_hip.stream_of(query))
    spruce_hip.check(rc, "spruce_selector_pool_project")
    return qp, kp


def project(x, W):
    """``x [..., D] @ W [D, P]`` in float32 with a sequential fused multiply-add over D."""
    _cuda(x, "x")
    if x.dtype != torch.float32 or W.dtype != torch.float32:
        raise ValueError("projection inputs must be float32")
    if W.dim() != 2 or x.shape[-1] != W.shape[0]:
        raise ValueError(f"shape mismatch: x {tuple(x.shape)} @ W {tuple(W.shape)}")
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    W = W.to(x.device).contiguous()
    N, D = x2.shape
    P = W.shape[1]
    out = torch.empty((N, P), device=x.device, dtype=torch.float32)
    with torch.cuda.device(x.device):
        rc = spruce_hip.lib().spruce_gate_project(
            spruce_hip.ptr(x2), spruce_hip.ptr(W), N, D, P, spruce_hip.ptr(out), spruce_hip.stream_of(x))
    spruce_hip.check(rc, "spruce_gate_project")
    return out.reshape(x.shape[:-1] + (P,))


def project_levels(levels, W, interleaved=False):
    """Projection of prototype rows kept in several buffers: ``levels`` is a
    list of ``[S, n_v, P, D]`` tensors (bf16, f16 or float32, one dtype; the
    levels of a key tree, leaf first) and the result is ``[S, sum n_v, P, p]``
    float32, level after level along the node axis.  The same values as
    ``project(torch.cat(levels, dim=1).float(), W)``, without the copies.
    ``interleaved=True`` returns the same values as ``[S, N, p/4, P, 4]``
    (each node's prototypes interleaved by 4-float group), the key layout
    the tree traversal reads fastest."""
    if not levels:
        raise ValueError("levels must not be empty")
    for t in levels:
        _cuda(t, "levels")
    S, _, P, D = levels[0].shape
    dtype = levels[0].dtype
    for t in levels:
        if t.dim() != 4 or t.shape[0] != S or t.shape[2:] != (P, D) or t.dtype != dtype:
            raise ValueError("levels must be [S, n, P, D] with one S, P, D and dtype")
    if W.dim() != 2 or W.shape[0] != D:
        raise ValueError(f"shape mismatch: levels [..., {D}] @ W {tuple(W.shape)}")
    W = W.to(device=levels[0].device, dtype=torch.float32).contiguous()
    bufs = [t.contiguous() for t in levels]
    nodes = [t.shape[1] for t in bufs]
    p = W.shape[1]
    if interleaved and p % 4:
        raise ValueError("the interleaved layout needs a projection dim divisible by 4")
    shape = (S, sum(nodes), p // 4, P, 4) if interleaved else (S, sum(nodes), P, p)
    out = torch.empty(shape, device=bufs[0].device, dtype=torch.float32)
    ptrs = (ctypes.c_void_p * len(bufs))(*[t.data_ptr() for t in bufs])
    counts = (ctypes.c_int64 * len(bufs))(*nodes)
    with torch.cuda.device(bufs[0].device):
        rc = spruce_hip.lib().spruce_gate_project_levels(
            ptrs, counts, len(bufs), S, P, D, spruce_hip.dtype_code(bufs[0]), spruce_hip.ptr(W), W.shape[1],
            spruce_hip.ptr(out), 1 if interleaved else 0, spruce_hip.stream_of(bufs[0]))
    spruce_hip.check(rc, "spruce_gate_project_levels")
    return out


def project_pair(xa, Wa, xb, Wb):
    """``project(xa, Wa), project(xb, Wb)`` in one launch (same results)."""
    _cuda(xa, "xa")
    _cuda(xb, "xb")
    for x, W in ((xa, Wa), (xb, Wb)):
        if x.dtype != torch.float32 or W.dtype != torch.float32:
            raise ValueError("projection inputs must be float32")
        if W.dim() != 2 or x.shape[-1] != W.shape[0]:
            raise ValueError(f"shape mismatch: x {tuple(x.shape)} @ W {tuple(W.shape)}")
    if Wa.shape != Wb.shape:
        raise ValueError("the two projections must share [D, P]")
    xa2 = xa.reshape(-1, xa.shape[-1]).contiguous()
    xb2 = xb.reshape(-1, xb.shape[-1]).contiguous()
    Wa = Wa.to(xa.device).contiguous()
    Wb = Wb.to(xa.device).contiguous()
    D, P = Wa.shape
    oa = torch.empty((xa2.shape[0], P), device=xa.device, dtype=torch.float32)
    ob = torch.empty((xb2.shape[0], P), device=xa.device, dtype=torch.float32)
    with torch.cuda.device(xa.device):
        rc = spruce_hip.lib().spruce_gate_project2(
            spruce_hip.ptr(xa2), spruce_hip.ptr(Wa), xa2.shape[0], spruce_hip.ptr(xb2), spruce_hip.ptr(Wb),
            xb2.shape[0], D, P, spruce_hip.ptr(oa), spruce_hip.ptr(ob), spruce_hip.stream_of(xa))
    spruce_hip.check(rc, "spruce_gate_project2")
    return oa.reshape(xa.shape[:-1] + (P,)), ob.reshape(xb.shape[:-1] + (P,))


def gate_scores(qp, kp, causal=True, div=None):
    """MaxSim scores ``[S, Qb, Kb]`` from projected prototypes ``qp [S,Qb,Pq,P]``
    and ``kp [S,Kb,Pk,P]``, divided by ``div`` (default sqrt(P)); with
    ``causal`` the entries above the diagonal are -inf.  ``causal="lower"``
    (Qb == Kb) computes only j <= i and leaves the entries above the diagonal
    unspecified, for consumers that read only the causal part."""
    _cuda(qp, "qp")
    if qp.dim() != 4 or kp.dim() != 4 or qp.shape[0] != kp.shape[0] or qp.shape[3] != kp.shape[3]:
        raise ValueError("qp must be [S,Qb,Pq,P] and kp [S,Kb,Pk,P]")
    if qp.dtype != torch.float32 or kp.dtype != torch.float32:
        raise ValueError("projected prototypes must be float32")
    qp = qp.contiguous()
    kp = kp.contiguous()
    S, Qb, Pq, P = qp.shape
    Kb, Pk = kp.shape[1], kp.shape[2]
    d = math.sqrt(P) if div is None else float(div)
    out = torch.empty((S, Qb, Kb), device=qp.device, dtype=torch.float32)
    with torch.cuda.device(qp.device):
        rc = spruce_hip.lib().spruce_gate_scores(
            spruce_hip.ptr(qp), spruce_hip.ptr(kp), S, Qb, Kb, Pq, Pk, P, d,
            2 if causal == "lower" else int(bool(causal)),
            spruce_hip.ptr(out), spruce_hip.stream_of(qp))
    spruce_hip.check(rc, "spruce_gate_scores")
    return out


def causal_topk_blocks(scores, k):
    """Row-wise causal top-k of ``scores [..., Qb, Kb]`` -> int32 ``[..., Qb, k]``
    ascending with -1 padding; ties go to the lower block index."""
    _cuda(scores, "scores")
    if scores.dtype != torch.float32:
        raise ValueError("scores must be float32")
    if k < 1:
        raise ValueError(f"k must be >= 1, got {k}")
    Qb, Kb = scores.shape[-2:]
    s = scores.reshape(-1, Qb, Kb).contiguous()
    R = s.shape[0]
    out = torch.empty((R, Qb, k), device=scores.device, dtype=torch.int32)
    with torch.cuda.device(scores.device):
        rc = spruce_hip.lib().spruce_causal_topk(
            spruce_hip.ptr(s), R, Qb, Kb, k, spruce_hip.ptr(out), spruce_hip.stream_of(scores))
    spruce_hip.check(rc, "spruce_causal_topk")
    return out.reshape(scores.shape[:-1] + (k,))


def fused_route_applies(query, key, Wq, Wk):
    """True when ``select_blocks_fused`` covers the shapes: head_dim
    128, projection dim 128 (one ``[128, 128]`` weight per side), bf16 or fp16
    inputs, at most 8 query heads per KV head and at most 1024 key blocks."""
    if query is None or key is None or query.dim() != 4 or key.dim() != 4:
        return False
    if Wq.shape != Wk.shape or Wq.dim() != 2 or Wq.dtype != torch.float32 or Wk.dtype != torch.float32:
        return False
    if query.dtype != key.dtype or query.dtype not in (torch.bfloat16, torch.float16):
        return False
    B, Hq, T, D = query.shape
    Hkv = key.shape[1]
    if key.shape[0] != B or key.shape[2:] != query.shape[2:] or Wq.shape[0] != D:
        return False
    return bool(spruce_hip.lib().spruce_select_flat_supported(Hq, Hkv, T, D, spruce_hip.dtype_code(query),
                                                               Wq.shape[1]))


def select_blocks_fused(query, key, Wq, Wk, top_k=32):
    """The flat selector in two launches: the key side (pool + project into a
    workspace), then one persistent kernel whose waves pool and project the
    next tile of query blocks while the others score and select the current
    one.  Same selected blocks as ``select_blocks`` (same operation order);
    shapes per ``fused_route_applies``.  Opt-in: on MI355X at T = 65536 with
    28 / 4 heads it takes about 0.175 ms against 0.160 ms for the four
    launches, because the scores of 4-row tiles re-read the projected keys
    and run at the unpacked float32 FMA rate."""
    _cuda(query, "query")
    _cuda(key, "key")
    if not fused_route_applies(query, key, Wq, Wk):
        raise ValueError("the fused selector route does not apply to these shapes / dtypes")
    if top_k < 1:
        raise ValueError(f"top_k must be >= 1, got {top_k}")
    B, Hq, T, D = query.shape
    Hkv = key.shape[1]
    P = Wq.shape[1]
    nb = (T + BLOCK - 1) // BLOCK
    Wq = Wq.to(query.device).contiguous()
    Wk = Wk.to(query.device).contiguous()
    lib = spruce_hip.lib()
    nbytes = lib.spruce_select_flat_workspace_bytes(B, Hkv, T, P)
    ws = torch.empty(nbytes // 4, device=query.device, dtype=torch.float32)
    out = torch.empty((B, Hkv, nb, top_k), device=query.device, dtype=torch.int32)
    with torch.cuda.device(query.device):
        rc = lib.spruce_select_flat(
            spruce_hip.ptr(query), spruce_hip.strides(query), spruce_hip.ptr(key), spruce_hip.strides(key),
            B, Hq, Hkv, T, D, spruce_hip.dtype_code(query), spruce_hip.ptr(Wq), spruce_hip.ptr(Wk), P,
            math.sqrt(P), top_k, spruce_hip.ptr(ws), nbytes, spruce_hip.ptr(out), spruce_hip.stream_of(query))
    spruce_hip.check(rc, "spruce_select_flat")
    return out[:, None]


def select_blocks(query, key, Wq, Wk, top_k=32, return_intermediates=False):
    """The flat selector over one layer.

    Pools Q (group mean, block mean) and K (block mean and max), projects them
    with ``Wq``/``Wk`` (``[D, P]`` float32), scores every causal (query block,
    key block) pair by MaxSim over the key summaries {mean, max}, and keeps the
    top ``top_k`` blocks per (KV head, query block).

    Returns ``selected`` int32 ``[B, 1, Hkv, nb, top_k]`` (the selected_blocks
    layout with one layer), or a dict with every intermediate when
    ``return_intermediates``.  Without intermediates, shapes that
    ``pool_project_applies`` covers pool and project in one launch (same
    values).
    """
    if not return_intermediates and pool_project_applies(query, key, Wq, Wk):
        qp, kp = pool_project(query, key, Wq, Wk)
        B, Hkv, nb, P = qp.shape
        sc = gate_scores(qp.reshape(B * Hkv, nb, 1, P), kp.reshape(B * Hkv, nb, 2, P), causal="lower")
        return causal_topk_blocks(sc, top_k).reshape(B, Hkv, nb, top_k)[:, None]
    q_mean, k_sum = pool_blocks(query, key)
    B, Hkv, nb, D = q_mean.shape
    if Wq.shape == Wk.shape:
        qp, kp = project_pair(q_mean, Wq, k_sum, Wk)   # [B,Hkv,nb,P], [B,Hkv,nb,2,P]
    else:
        qp, kp = project(q_mean, Wq), project(k_sum, Wk)
    P = qp.shape[-1]
    # The top-k reads only j <= i; the intermediates keep the -inf fill.
    sc = gate_scores(qp.reshape(B * Hkv, nb, 1, P), kp.reshape(B * Hkv, nb, 2, P),
                     causal=True if return_intermediates else "lower")
    sel = causal_topk_blocks(sc, top_k).reshape(B, Hkv, nb, top_k)[:, None]
    if not return_intermediates:
        return sel
    return {"q_mean": q_mean, "k_sum": k_sum, "qp": qp, "kp": kp,
            "scores": sc.reshape(B, Hkv, nb, nb), "selected": sel}
