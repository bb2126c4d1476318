"""Block attention mass without the [T, T] matrix, on gfx950.

Drop-in for chunked_pool (teacher/chunked_extract.py:91-131 in the reference):
``chunked_pool(query, key, scaling, block_size=64, head_chunk=None)`` returns
``[b, H, q_blocks, k_blocks]`` float32 equal to
pool_attention(causal_softmax(q k^T * scaling)).  ``key`` may be repeated to H
heads as the reference passes it, or stay at native KV resolution
``[b, Hkv, k, d]`` (query head h reads KV head h // (H / Hkv)) -- no GQA copy
is needed.  Two HIP passes (row statistics, then tile mass) behind the C ABI;
``head_chunk`` is accepted for signature compatibility and ignored (nothing
is materialised per head).
"""
import torch

import spruce_hip

_BLOCK = 64


@torch.no_grad()
def chunked_pool(query, key, scaling, block_size=_BLOCK, head_chunk=None):
    del head_chunk
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
    nbytes = spruce_hip.lib().spruce_teacher_workspace_bytes(b, H, q_len)
    ws = torch.empty(nbytes // 4, device=query.device, dtype=torch.float32)
    with torch.cuda.device(query.device):
        rc = spruce_hip.lib().spruce_teacher_block_mass(
            spruce_hip.ptr(query), spruce_hip.strides(query), spruce_hip.ptr(key), spruce_hip.strides(key),
            b, H, Hkv, q_len, d, float(scaling), spruce_hip.dtype_code(query),
            spruce_hip.ptr(mass), spruce_hip.ptr(ws), nbytes, spruce_hip.stream_of(query))
    spruce_hip.check(rc, "spruce_teacher_block_mass")
    return mass
