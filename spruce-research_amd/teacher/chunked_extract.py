"""Block attention mass without the [T, T] matrix, on gfx950.

Drop-in for chunked_pool (teacher/chunked_extract.py:91-131 in the reference):
``chunked_pool(query, key, scaling, block_size=64, head_chunk=None)`` returns
``[b, H, q_blocks, k_blocks]`` float32 equal to
pool_attention(causal_softmax(q k^T * scaling)).  ``key`` may be repeated to H
heads as the reference passes it, or stay at native KV resolution
``[b, Hkv, k, d]`` (query head h reads KV head h // (H / Hkv)) -- no GQA copy
is needed.  One HIP kernel computes QK^T once per causal tile (online row
statistics plus per-row partial sums of every key block in a workspace,
combined once each row is complete); sequences whose workspace partials would
exceed 4 GiB use two passes (row statistics, then recomputed tile mass).  ``head_chunk`` is
accepted for signature compatibility and ignored (nothing is materialised
per head).

Selector prototype features (teacher/chunked_extract.py:27-80 in the
reference), in the model dtype: ``_group_avg_tokens(x, G)`` and
``_proto_pool_seq(x, block, P)`` with the reference's signatures, plus
``proto_pool_grouped(query, G, block, P)``, which fuses the two (the per-token
group average never goes to HBM).  Prototype 0 is the mean of the block's
real rows; prototypes 1..P-1 are the rows farthest from it in float32 squared
L2 (farthest first, ties to the lower row), and slots past the real rows hold
the mean.
"""
import torch
import torch.nn.functional as F

import spruce_hip
from spruce_hip.overlay import forward_missing

__getattr__ = forward_missing("teacher.chunked_extract", __file__)

_BLOCK = 64
_PROTO = 8


@torch.no_grad()
def chunked_pool(query, key, scaling, block_size=_BLOCK, head_chunk=None):
    del head_chunk
    return block_mass(query, key, scaling, block_size=block_size)


_SCHEDULES = {"auto": 0, "scratch": 1, "two_pass": 2}


def block_mass(query, key, scaling, block_size=_BLOCK, schedule="auto"):
    """chunked_pool's computation.  ``schedule``: "auto" (the single pass
    when its workspace partials take at most 4 GiB), "scratch" (single pass)
    or "two_pass"."""
    if schedule not in _SCHEDULES:
        raise ValueError(f"schedule must be one of {tuple(_SCHEDULES)}, got {schedule!r}")
    if block_size != _BLOCK:
        raise ValueError("the HIP block-mass kernel requires block_size=64")
    if not query.is_cuda:
        raise RuntimeError("chunked_pool (HIP) requires GPU tensors")
    if query.dim() != 4 or key.dim() != 4:
        raise ValueError("query and key must be [b, heads, tokens, head_dim]")
    b, H, q_len, d = query.shape
    if key.shape[0] != b or key.shape[3] != d or key.shape[1] == 0 or H % key.shape[1]:
        raise ValueError("key must be [b, H or a divisor of H, k_len, head_dim]")
    if key.shape[2] != q_len:
        raise ValueError("prefill teacher extraction needs q_len == k_len")
    if key.dtype != query.dtype:
        raise ValueError("query and key must share a dtype")
    Hkv = key.shape[1]
    qb = (q_len + _BLOCK - 1) // _BLOCK
    mass = torch.empty((b, H, qb, qb), device=query.device, dtype=torch.float32)
    lib = spruce_hip.lib()
    code = _SCHEDULES[schedule]
    if code == 0:
        code = lib.spruce_teacher_schedule(b, H, Hkv, q_len, d, spruce_hip.SIZE_MAX)
        spruce_hip.check(code if code < 0 else 0, "spruce_teacher_schedule")
    nbytes = lib.spruce_teacher_schedule_workspace_bytes(b, H, q_len, code)
    ws = torch.empty((nbytes + 3) // 4, device=query.device, dtype=torch.float32)
    with torch.cuda.device(query.device):
        rc = lib.spruce_teacher_block_mass_schedule(
            spruce_hip.ptr(query), spruce_hip.strides(query), spruce_hip.ptr(key), spruce_hip.strides(key),
            b, H, Hkv, q_len, d, float(scaling), spruce_hip.dtype_code(query),
            spruce_hip.ptr(mass), spruce_hip.ptr(ws), nbytes, code, spruce_hip.stream_of(query))
    spruce_hip.check(rc, "spruce_teacher_block_mass")
    return mass


def _features_input(x, name):
    if not x.is_cuda:
        raise RuntimeError(f"{name} (HIP) requires GPU tensors")
    if x.dim() != 4:
        raise ValueError(f"{name} expects [b, H, L, d], got {tuple(x.shape)}")


def _launch_proto(x, G, block, P):
    b, H, L, d = x.shape
    if H % G:
        raise ValueError(f"H={H} not divisible by G={G}")
    if not 1 <= block <= 64:
        raise ValueError(f"the HIP prototype kernel supports 1 <= block <= 64, got {block}")
    if d > 128:
        raise ValueError(f"the HIP prototype kernel supports head_dim <= 128, got {d}")
    if x.stride(-1) == 1 and d % 8 == 0 and (x.data_ptr() % 16 or any((s * x.element_size()) % 16 for s in x.stride()[:3])):
        x = x.contiguous()
    nb = (L + block - 1) // block
    out = torch.empty((b, G, nb, P, d), device=x.device, dtype=x.dtype)
    if out.numel() == 0:
        return out
    with torch.cuda.device(x.device):
        rc = spruce_hip.lib().spruce_proto_pool(
            spruce_hip.ptr(x), spruce_hip.strides(x), b, H, L, d, G, block, P,
            spruce_hip.dtype_code(x), spruce_hip.ptr(out), spruce_hip.stream_of(x))
    spruce_hip.check(rc, "spruce_proto_pool")
    return out


@torch.no_grad()
def _proto_pool_seq(x, block, P):
    """[b,H,L,d] -> [b,H,nb,P,d]: P prototype vectors per block (mean + P-1 outliers)."""
    _features_input(x, "_proto_pool_seq")
    return _launch_proto(x, x.shape[1], block, P)


@torch.no_grad()
def proto_pool_grouped(query, G, block=_BLOCK, P=_PROTO):
    """_proto_pool_seq(_group_avg_tokens(query, G), block, P) in one kernel: [b,H,L,d] -> [b,G,nb,P,d]."""
    _features_input(query, "proto_pool_grouped")
    return _launch_proto(query, G, block, P)


def _aligned16(x):
    return x.data_ptr() % 16 == 0 and all((s * x.element_size()) % 16 == 0 for s in x.stride()[:3])


@torch.no_grad()
def proto_pool_qk(query, key, block=_BLOCK, P=_PROTO):
    """``(proto_pool_grouped(query, G, block, P), _proto_pool_seq(key, block, P))``
    with G = key's head count, in one launch when both are 16-bit with
    16-byte aligned rows, head_dim a multiple of 8 up to 128 and at most 8
    query heads per KV head (each block's key loads then overlap its query
    work); otherwise the two launches.  The same values either way."""
    _features_input(query, "proto_pool_qk")
    _features_input(key, "proto_pool_qk")
    b, H, L, d = query.shape
    G = key.shape[1]
    if key.shape[0] != b or key.shape[2:] != query.shape[2:] or H % G:
        raise ValueError(f"key {tuple(key.shape)} does not match query {tuple(query.shape)}")
    fused = (query.dtype == key.dtype and query.dtype in (torch.bfloat16, torch.float16) and d % 8 == 0
             and d <= 128 and H // G <= 8 and 1 <= block <= 64 and query.stride(-1) == 1 and key.stride(-1) == 1
             and _aligned16(query) and _aligned16(key))
    if not fused:
        return proto_pool_grouped(query, G, block, P), _proto_pool_seq(key, block, P)
    nb = (L + block - 1) // block
    out_q = torch.empty((b, G, nb, P, d), device=query.device, dtype=query.dtype)
    out_k = torch.empty((b, G, nb, P, d), device=query.device, dtype=query.dtype)
    with torch.cuda.device(query.device):
        rc = spruce_hip.lib().spruce_proto_pool_qk(
            spruce_hip.ptr(query), spruce_hip.strides(query), spruce_hip.ptr(key), spruce_hip.strides(key),
            b, H, G, L, d, block, P, spruce_hip.dtype_code(query), spruce_hip.ptr(out_q), spruce_hip.ptr(out_k),
            spruce_hip.stream_of(query))
    spruce_hip.check(rc, "spruce_proto_pool_qk")
    return out_q, out_k


@torch.no_grad()
def _group_avg_tokens(x, G):
    """[b,H,L,d] -> [b,G,L,d]: the H/G query heads of each KV group averaged per token."""
    _features_input(x, "_group_avg_tokens")
    b, H, L, d = x.shape
    if H % G:
        raise AssertionError(f"H={H} not divisible by G={G}")
    if x.stride(-1) == 1 and d % 8 == 0 and (x.data_ptr() % 16 or any((s * x.element_size()) % 16 for s in x.stride()[:3])):
        x = x.contiguous()
    out = torch.empty((b, G, L, d), device=x.device, dtype=x.dtype)
    if out.numel() == 0:
        return out
    with torch.cuda.device(x.device):
        rc = spruce_hip.lib().spruce_group_avg_tokens(
            spruce_hip.ptr(x), spruce_hip.strides(x), b, H, L, d, G,
            spruce_hip.dtype_code(x), spruce_hip.ptr(out), spruce_hip.stream_of(x))
    spruce_hip.check(rc, "spruce_group_avg_tokens")
    return out


@torch.no_grad()
def causal_prefill_features(query, key, value, scaling, P=_PROTO, capture=True):
    """Dense causal GQA attention of the capture hooks with the selector
    features as a by-product of the same HIP pass (``spruce_causal_prefill``).

    query ``[b,H,L,d]`` (any strides with a contiguous last dim, e.g. the
    transposed view of a ``[b,L,H,d]`` projection); key/value ``[b,G,L,d]`` at
    KV-head resolution (no repeat).  Returns ``(attn_output, pooled_q,
    pooled_k)``: attn_output ``[b,L,H,d]`` contiguous (what the hooks return,
    teacher/chunked_extract.py:155-161 in the reference), pooled_q =
    ``_proto_pool_seq(_group_avg_tokens(query, G), 64, P)`` and pooled_k =
    ``_proto_pool_seq(key, 64, P)`` (:145-147), bit for bit the standalone
    kernels' results.  The attention kernel writes the group-averaged query
    tokens and the key prototypes while it holds the tiles; one small launch
    pools the grouped queries.  ``capture=False`` runs the attention only
    (pooled_* are None).
    """
    from kernels.direct_index import _check_common, _output
    B, H, G, L, d = _check_common(query, key, value, _BLOCK, "tiled_gqa")
    if any(x.stride(-1) != 1 for x in (query, key, value)):
        raise ValueError("query, key and value must have a contiguous final dimension")
    q_grouped = k_protos = None
    if capture:
        if query.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError(f"feature capture runs in the model dtype (bf16 or f16), got {query.dtype}")
        if H // G > 8:
            raise ValueError(f"feature capture supports at most 8 query heads per KV head, got {H // G}")
        if not 1 <= P <= 65:
            raise ValueError(f"P must be in [1, 65], got {P}")
        nb = (L + _BLOCK - 1) // _BLOCK
        q_grouped = torch.empty((B, G, L, d), device=query.device, dtype=query.dtype)
        k_protos = torch.empty((B, G, nb, P, d), device=query.device, dtype=query.dtype)
    out, out_strides = _output(query)
    with torch.cuda.device(query.device):
        rc = spruce_hip.lib().spruce_causal_prefill(
            spruce_hip.ptr(query), spruce_hip.strides(query), spruce_hip.ptr(key), spruce_hip.strides(key),
            spruce_hip.ptr(value), spruce_hip.strides(value), B, H, G, L, d, float(scaling),
            spruce_hip.dtype_code(query), spruce_hip.ptr(out), out_strides,
            spruce_hip.ptr(q_grouped), spruce_hip.ptr(k_protos), P, spruce_hip.stream_of(query))
    spruce_hip.check(rc, "spruce_causal_prefill")
    if not capture:
        return out, None, None
    return out, _launch_proto(q_grouped, G, _BLOCK, P), k_protos


def _fused_capture_ok(query, key, value, dropout):
    # The fused pass covers the hooks' deployed settings; anything else keeps
    # the separate prototype kernels plus torch's fused SDPA, as the reference.
    return (_BLOCK == 64 and not dropout and query.dtype in (torch.bfloat16, torch.float16)
            and query.shape[-1] in (64, 128) and query.shape[1] % key.shape[1] == 0
            and query.shape[1] // key.shape[1] <= 8
            and query.stride(-1) == 1 and key.stride(-1) == 1 and value.stride(-1) == 1)


# ---------------------------------------------------------------------------
# Hugging Face capture hooks (teacher/chunked_extract.py:134-265 in the reference).
# The attention function computes the teacher mass (HIP chunked_pool at native
# KV resolution: no repeated K copy), then propagates the layer through the HIP
# dense causal kernel, which emits the selector prototypes from the same pass
# (bf16/f16, head_dim 64/128, at most 8 query heads per KV head, no dropout;
# other settings keep the standalone prototype kernels and torch's fused causal
# SDPA, as the reference).

# layer_idx -> pooled mass [1, H, qb, kb] (cpu, float32)
_CAPTURE = {}
# layer_idx -> (pooledQ [1, G, qb, P, d], pooledK [1, G, kb, P, d]) (cpu, model dtype)
_CAPTURE_QK = {}
_REGISTERED = False
_FEATURES_REGISTERED = False


def _repeat_kv(x, n_rep):
    if n_rep == 1:
        return x
    b, h, t, d = x.shape
    return x[:, :, None].expand(b, h, n_rep, t, d).reshape(b, h * n_rep, t, d)


def _propagate(query, key, value, scaling, dropout):
    n_rep = query.shape[1] // key.shape[1]
    out = F.scaled_dot_product_attention(
        query, _repeat_kv(key, n_rep), _repeat_kv(value, n_rep),
        attn_mask=None, dropout_p=dropout, scale=scaling, is_causal=True)
    return out.transpose(1, 2).contiguous()


def _capture_qk(module, query, key):
    pooled_q, pooled_k = proto_pool_qk(query, key, _BLOCK, _PROTO)
    _CAPTURE_QK[module.layer_idx] = (pooled_q.cpu(), pooled_k.cpu())


def _capture_fused(module, query, key, value, scaling):
    out, pooled_q, pooled_k = causal_prefill_features(query, key, value, scaling, _PROTO)
    _CAPTURE_QK[module.layer_idx] = (pooled_q.cpu(), pooled_k.cpu())
    return out


def _capture_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0,
                       sliding_window=None, **kwargs):
    """Attention function "chunked_capture": records mass and prototypes for the layer."""
    if scaling is None:
        scaling = query.shape[-1] ** -0.5
    _CAPTURE[module.layer_idx] = chunked_pool(query, key, scaling, _BLOCK).cpu()
    if _fused_capture_ok(query, key, value, dropout):
        return _capture_fused(module, query, key, value, scaling), None
    _capture_qk(module, query, key)
    return _propagate(query, key, value, scaling, dropout), None


def _capture_features(module, query, key, value, attention_mask, scaling=None, dropout=0.0,
                      sliding_window=None, **kwargs):
    """Attention function "selector_feature_capture": prototypes only, no teacher mass."""
    if scaling is None:
        scaling = query.shape[-1] ** -0.5
    if _fused_capture_ok(query, key, value, dropout):
        return _capture_fused(module, query, key, value, scaling), None
    _capture_qk(module, query, key)
    return _propagate(query, key, value, scaling, dropout), None


def _ensure_registered():
    global _REGISTERED
    if not _REGISTERED:
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
        ALL_ATTENTION_FUNCTIONS.register("chunked_capture", _capture_attention)
        _REGISTERED = True


def _ensure_features_registered():
    global _FEATURES_REGISTERED
    if not _FEATURES_REGISTERED:
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
        ALL_ATTENTION_FUNCTIONS.register("selector_feature_capture", _capture_features)
        _FEATURES_REGISTERED = True


def _stack_and_clear_captures(order):
    """Stack one prompt's per-layer captures along a layer axis, then drop them."""
    try:
        return (torch.stack([_CAPTURE[i] for i in order], dim=1),
                torch.stack([_CAPTURE_QK[i][0] for i in order], dim=1),
                torch.stack([_CAPTURE_QK[i][1] for i in order], dim=1))
    finally:
        _CAPTURE.clear()
        _CAPTURE_QK.clear()


def _set_attn_impl(model, name):
    model.config._attn_implementation = name
    for m in model.modules():
        cfg = getattr(m, "config", None)
        if cfg is not None:
            cfg._attn_implementation = name


@torch.no_grad()
def get_pooled_targets(model, tok, prompt, device="cuda", block_size=_BLOCK):
    """One forward of the base decoder capturing, per layer, the pooled teacher mass and
    the selector prototypes.  Returns (pooled [1, L, H, qb, kb] float32 cpu,
    pooledQ [1, L, G, qb, P, d] and pooledK [1, L, G, kb, P, d] in the model dtype on
    cpu, seq_len)."""
    if block_size != _BLOCK:
        raise ValueError("the HIP teacher kernels use block_size=64")
    _ensure_registered()
    _CAPTURE.clear()
    _CAPTURE_QK.clear()
    prev = model.config._attn_implementation
    _set_attn_impl(model, "chunked_capture")
    try:
        inputs = tok(prompt, return_tensors="pt").to(device)
        model.model(**inputs, use_cache=False)
    finally:
        _set_attn_impl(model, prev)
    seq_len = inputs["input_ids"].shape[1]
    pooled, pooled_q, pooled_k = _stack_and_clear_captures(sorted(_CAPTURE))
    return pooled, pooled_q, pooled_k, seq_len


@torch.no_grad()
def get_selector_features(model, tok, prompt, device="cuda", block_size=_BLOCK):
    """One forward of the base decoder capturing only the selector prototypes
    (no teacher mass): returns (pooledQ [1, L, G, qb, P, d], pooledK
    [1, L, G, kb, P, d], both in the model dtype on cpu, seq_len), like the
    reference's get_selector_features (teacher/chunked_extract.py:268-311)."""
    if block_size != _BLOCK:
        raise ValueError("the HIP teacher kernels use block_size=64")
    _ensure_features_registered()
    _CAPTURE.clear()
    _CAPTURE_QK.clear()
    prev = model.config._attn_implementation
    _set_attn_impl(model, "selector_feature_capture")
    try:
        inputs = tok(prompt, return_tensors="pt").to(device)
        model.model(**inputs, use_cache=False)
    finally:
        _set_attn_impl(model, prev)
    try:
        order = sorted(_CAPTURE_QK)
        pooled_q = torch.stack([_CAPTURE_QK[i][0] for i in order], dim=1)
        pooled_k = torch.stack([_CAPTURE_QK[i][1] for i in order], dim=1)
    finally:
        _CAPTURE.clear()
        _CAPTURE_QK.clear()
    return pooled_q, pooled_k, inputs["input_ids"].shape[1]
