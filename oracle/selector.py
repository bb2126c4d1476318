"""Selector oracle (ctypes wrapper of oracle/selector.c and oracle/proto.c) -- TEST INFRASTRUCTURE ONLY.

The C code fixes the exact float32 operation order the HIP selector kernels
follow, so pooled summaries, projections, scores and the selected block
indices are comparable bit for bit.  Reference semantics (file:line in the
reference) are listed in oracle/selector.c.
"""
import ctypes
import math
import os

import numpy as np

_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_build", "liboracle_selector.so")
_lib = None

BLOCK = 64

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            raise RuntimeError(f"{_LIB} missing; run `make -C oracle`")
        h = ctypes.CDLL(_LIB)
        ci = ctypes.c_int
        h.oracle_block_pool.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ci, ci, ci, ci, ci,
                                        ctypes.c_void_p, ctypes.c_void_p]
        h.oracle_project.argtypes = [_f32p, _f32p, ci, ci, ci, _f32p]
        h.oracle_scores.argtypes = [_f32p, _f32p, ci, ci, ci, ci, ci, ci, ctypes.c_float, ci, _f32p]
        h.oracle_topk.argtypes = [_f32p, ci, ci, ci, ci, _i32p]
        h.oracle_round.argtypes = [_f32p, ctypes.c_int64, ci, _f32p]
        h.oracle_group_avg.argtypes = [_f32p, ci, ci, ci, ci, ci, ci, _f32p]
        h.oracle_proto_pool.argtypes = [_f32p, ci, ci, ci, ci, ci, ci, ci, _f32p]
        for f in (h.oracle_block_pool, h.oracle_project, h.oracle_scores, h.oracle_topk,
                  h.oracle_round, h.oracle_group_avg, h.oracle_proto_pool):
            f.restype = None
        _lib = h
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def block_pool(q, k):
    """q [B,Hq,T,D], k [B,Hkv,T,D] (float32-representable values).

    Returns (q_mean [B,Hkv,nb,D], k_sum [B,Hkv,nb,2,D] with proto 0 = mean,
    proto 1 = per-dim max)."""
    q = None if q is None else np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    B, Hkv, T, D = k.shape
    Hq = q.shape[1] if q is not None else Hkv
    nb = (T + BLOCK - 1) // BLOCK
    q_mean = np.zeros((B, Hkv, nb, D), np.float32)
    k_sum = np.zeros((B, Hkv, nb, 2, D), np.float32)
    lib().oracle_block_pool(_ptr(q), _ptr(k), B, Hq, Hkv, T, D, _ptr(q_mean), _ptr(k_sum))
    return q_mean, k_sum


def project(x, W):
    """x [..., D] @ W [D, P] with a sequential fmaf chain over D."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    D, P = W.shape
    flat = x.reshape(-1, D)
    out = np.zeros((flat.shape[0], P), np.float32)
    lib().oracle_project(flat, W, flat.shape[0], D, P, out)
    return out.reshape(x.shape[:-1] + (P,))


def scores(qp, kp, div=None, causal=True):
    """qp [BG,Qb,Pq,P], kp [BG,Kb,Pk,P] -> MaxSim scores [BG,Qb,Kb] (-inf above the diagonal if causal)."""
    qp = np.ascontiguousarray(qp, dtype=np.float32)
    kp = np.ascontiguousarray(kp, dtype=np.float32)
    BG, Qb, Pq, P = qp.shape
    Kb, Pk = kp.shape[1], kp.shape[2]
    d = np.float32(math.sqrt(P)) if div is None else np.float32(div)
    out = np.zeros((BG, Qb, Kb), np.float32)
    lib().oracle_scores(qp, kp, BG, Qb, Kb, Pq, Pk, P, float(d), int(causal), out)
    return out


def topk(s, k):
    """s [R,Qb,Kb] -> int32 [R,Qb,k]: causal top-k, ties to the lower index, ascending, -1 pad."""
    s = np.ascontiguousarray(s, dtype=np.float32)
    R, Qb, Kb = s.shape
    out = np.zeros((R, Qb, k), np.int32)
    lib().oracle_topk(s, R, Qb, Kb, k, out)
    return out


def flat_select(q, k, Wq, Wk, top_k=32):
    """The whole cfg3 front end: pooled Q (group mean, block mean), K mean and
    max summaries, projections, MaxSim scores over {mean, max}, causal top-k.

    q [B,Hq,T,D], k [B,Hkv,T,D]; Wq, Wk [D, P].  Returns a dict with every
    intermediate and ``selected`` int32 [B, 1, Hkv, nb, top_k]."""
    q_mean, k_sum = block_pool(q, k)
    B, Hkv, nb, D = q_mean.shape
    qp = project(q_mean, Wq)[:, :, :, None, :]          # [B,Hkv,nb,1,P]
    kp = project(k_sum, Wk)                              # [B,Hkv,nb,2,P]
    P = Wq.shape[1]
    sc = scores(qp.reshape(B * Hkv, nb, 1, P), kp.reshape(B * Hkv, nb, 2, P))
    sel = topk(sc, top_k)
    return {"q_mean": q_mean, "k_sum": k_sum, "qp": qp, "kp": kp,
            "scores": sc.reshape(B, Hkv, nb, nb),
            "selected": sel.reshape(B, Hkv, nb, top_k)[:, None]}


DTYPE_CODES = {"bfloat16": 0, "float16": 1, "float32": 2}


def round_to(x, dtype):
    """Nearest-even rounding of float32 values to the model dtype ("bfloat16", "float16", "float32")."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().oracle_round(x.reshape(-1), x.size, DTYPE_CODES[dtype], out.reshape(-1))
    return out


def group_avg(x, G, dtype):
    """x [B,H,L,D] (model-dtype values as float32) -> [B,G,L,D] (_group_avg_tokens)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    B, H, L, D = x.shape
    if H % G:
        raise ValueError(f"H={H} not divisible by G={G}")
    out = np.zeros((B, G, L, D), np.float32)
    lib().oracle_group_avg(x, B, H, L, D, G, DTYPE_CODES[dtype], out)
    return out


def proto_pool(a, block, P, dtype):
    """a [B,G,L,D] -> [B,G,nb,P,D]: mean + the min(P-1, block) farthest rows (_proto_pool_seq)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    B, G, L, D = a.shape
    if block > 64 or D > 512:
        raise ValueError("oracle proto_pool supports block <= 64 and D <= 512")
    nb = (L + block - 1) // block
    out = np.zeros((B, G, nb, P, D), np.float32)
    lib().oracle_proto_pool(a, B, G, L, D, block, P, DTYPE_CODES[dtype], out)
    return out
