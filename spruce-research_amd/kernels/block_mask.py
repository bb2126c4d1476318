"""Block-mask causal sparse prefill on gfx950 (HIP, C ABI).

Host side of ``spruce_sparse_prefill_mask``.  Mirrors the reference's
``block_sparse_triton(q, k, v, block_mask, scale, block_size=64)``
(kernels/seerattention_triton.py:71-90): q/k/v are ``[B,H,T,D]``, the mask is
``[B,H,ceil(T/64),ceil(T/64)]`` bool, only columns ``0..query_block`` of a row
are read, and the output is a contiguous ``[B,H,T,D]`` tensor like
``torch.empty_like(q)``.

Unlike the reference kernel, K/V may stay at native GQA resolution
(``[B,Hkv,T,D]`` with ``Hq % Hkv == 0``) and the mask may be given per query
head (``Hm == Hq``, the layout of ``selected_blocks_to_block_mask``) or per KV
head (``Hm == Hkv``); no input is copied or expanded.
"""
import torch

import spruce_hip


def block_sparse_prefill(q, k, v, block_mask, scale, block_size=64,
                         kernel_variant="single_head"):
    if not q.is_cuda:
        raise RuntimeError("the block-mask HIP backend requires GPU tensors")
    if block_size != 64:
        raise ValueError("the block-mask kernel currently supports block_size=64 only")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, and v must be [B,H,T,D]")
    if k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[2:] != k.shape[2:]:
        raise ValueError("q, k, and v must have matching [B,H,T,D] shapes")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k and v must share one dtype")
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    if Hq % Hkv:
        raise ValueError("query heads must be divisible by KV heads")
    if D not in (64, 128):
        raise ValueError(f"kernel supports head_dim 64 or 128, got {D}")
    qblocks = (T + block_size - 1) // block_size
    if block_mask.dim() != 4 or block_mask.shape[0] != B or block_mask.shape[2] != qblocks \
            or block_mask.shape[3] < qblocks:
        raise ValueError("block_mask must be [B,H,ceil(T/64),ceil(T/64)]")
    Hm = block_mask.shape[1]
    if Hm not in (Hq, Hkv):
        raise ValueError("block_mask heads must equal query heads or KV heads")
    if block_mask.dtype not in (torch.bool, torch.uint8):
        raise ValueError("block_mask must be bool")
    if any(x.stride(-1) != 1 for x in (q, k, v)):
        raise ValueError("q, k, and v must have a contiguous final dimension")
    if block_mask.device != q.device:
        raise ValueError("block_mask must be on the same device as q")
    mask_u8 = block_mask.view(torch.uint8) if block_mask.dtype == torch.bool else block_mask
    out = torch.empty((B, Hq, T, D), device=q.device, dtype=q.dtype)
    with torch.cuda.device(q.device):
        rc = spruce_hip.lib().spruce_sparse_prefill_mask(
            spruce_hip.ptr(q), spruce_hip.strides(q),
            spruce_hip.ptr(k), spruce_hip.strides(k),
            spruce_hip.ptr(v), spruce_hip.strides(v),
            spruce_hip.ptr(mask_u8), spruce_hip.strides(mask_u8), Hm,
            B, Hq, Hkv, T, D, float(scale), spruce_hip.dtype_code(q),
            spruce_hip.variant_code(kernel_variant),
            spruce_hip.ptr(out), spruce_hip.strides(out), spruce_hip.stream_of(q))
    spruce_hip.check(rc, "spruce_sparse_prefill_mask")
    return out
