"""Direct-index block-sparse causal GQA prefill on gfx950 (HIP, C ABI).

Host side of ``spruce_sparse_prefill_index`` / ``spruce_sparse_prefill_csr``.
It mirrors the reference's ``direct_index_sparse_triton``
(kernels/seerattention_direct_index_triton.py:339-416): the same argument
meaning, validation order, exception types and output layout -- q is
``[B,Hq,T,D]`` (any strides with a contiguous last dim, e.g. the transposed
view of Qwen's ``[B,T,Hq,D]`` projection), k/v and indices stay at KV-head
resolution, and the output is a contiguous ``[B,T,Hq,D]`` tensor written
through logical ``[B,Hq,T,D]`` strides.
"""
import torch

import spruce_hip
from spruce_hip import KERNEL_VARIANTS

_LAST_CONFIG = {}


def _check_common(q, k, v, block_size, kernel_variant):
    if kernel_variant not in KERNEL_VARIANTS:
        raise ValueError(
            f"kernel_variant must be one of {KERNEL_VARIANTS}, "
            f"got {kernel_variant!r}")
    if not q.is_cuda:
        raise RuntimeError("the direct-index HIP backend requires GPU tensors")
    if block_size != 64:
        raise ValueError("direct-index kernel currently supports block_size=64 only")
    if k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[2:] != k.shape[2:]:
        raise ValueError("q and k/v must match in batch, tokens, and head_dim")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k and v must share one dtype")
    if k.device != q.device or v.device != q.device:
        raise ValueError("q, k and v must be on the same device")
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    if Hq % Hkv:
        raise ValueError("query heads must be divisible by KV heads")
    if D not in (64, 128):
        raise ValueError(f"kernel supports head_dim 64 or 128, got {D}")
    return B, Hq, Hkv, T, D


def _output(q):
    B, Hq, T, D = q.shape
    out = torch.empty((B, T, Hq, D), device=q.device, dtype=q.dtype)
    # Logical [B,Hq,T,D] strides over the contiguous [B,T,Hq,D] storage.
    return out, spruce_hip.strides(out, order=(0, 2, 1, 3))


def _record(kernel_variant, Hq, Hkv, D):
    _LAST_CONFIG[kernel_variant] = spruce_hip.launch_config(
        kernel_variant, Hq, Hkv, D)["best_config"]


def _key_valid(key_valid, B, T, device):
    """bool/uint8 ``[B, T]`` key validity -> contiguous uint8 on ``device``."""
    if key_valid.shape != (B, T):
        raise ValueError(f"key_valid must be [B, T] = {(B, T)}, got {tuple(key_valid.shape)}")
    if key_valid.device != device:
        raise ValueError("key_valid must be on the same device as q")
    return key_valid.to(torch.bool).contiguous().view(torch.uint8)


_MASK_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2, torch.bool: 3}


def _attn_mask(mask, B, Hq, T, device):
    """A 4-D attention mask ``[B, 1 or Hq, >=T, >=T]`` as (tensor, dtype code),
    last dimension contiguous; bool stays bool (read as bytes), other float
    types go to float32."""
    if mask.dim() != 4:
        raise ValueError(f"attn_mask must be 4-D [B, Hm, T, T], got {tuple(mask.shape)}")
    if mask.shape[0] != B or mask.shape[1] not in (1, Hq) or mask.shape[2] < T or mask.shape[3] < T:
        raise ValueError(f"attn_mask {tuple(mask.shape)} does not cover batch {B}, 1 or {Hq} heads and "
                         f"{T} query/key tokens")
    if mask.device != device:
        raise ValueError("attn_mask must be on the same device as q")
    if mask.dtype not in _MASK_DTYPES:
        mask = mask.float()
    if mask.stride(-1) != 1:
        mask = mask.contiguous()
    return mask, _MASK_DTYPES[mask.dtype]


def direct_index_sparse_prefill(q, k, v, indices, scale, block_size=64,
                                kernel_variant="single_head", key_valid=None, attn_mask=None):
    """Causal block-sparse attention over exactly the supplied block IDs.

    indices: int32 ``[B,Hkv,ceil(T/64),K]``; negative entries are padding.
    key_valid: optional bool ``[B,T]`` key padding (False keys get no weight;
    a query row with no valid causal listed key writes zeros).
    attn_mask: optional 4-D mask ``[B, 1 or Hq, T, T]`` over (query, key)
    tokens, added to the scaled scores of the listed causal keys as the
    reference's PyTorch path does (sparse/attention.py:223-229): a float mask
    is added (0 attends, -inf / finfo.min gives no weight), a bool mask
    attends where True.  A query row with no surviving key writes zeros.
    Returns ``[B,T,Hq,D]`` in q's dtype.
    """
    B, Hq, Hkv, T, D = _check_common(q, k, v, block_size, kernel_variant)
    qblocks = (T + block_size - 1) // block_size
    if tuple(indices.shape[:3]) != (B, Hkv, qblocks) or indices.dtype != torch.int32:
        raise ValueError("indices must be int32 [B,Hkv,ceil(T/64),K]")
    if indices.dim() != 4:
        raise ValueError("indices must be int32 [B,Hkv,ceil(T/64),K]")
    if any(x.stride(-1) != 1 for x in (q, k, v, indices)):
        raise ValueError("q, k, v, and indices must have a contiguous final dimension")
    if indices.device != q.device:
        raise ValueError("indices must be on the same device as q")
    out, out_strides = _output(q)
    if attn_mask is not None:
        if key_valid is not None:
            raise ValueError("pass either key_valid or attn_mask, not both")
        mask, code = _attn_mask(attn_mask, B, Hq, T, q.device)
        mview = mask.view(torch.uint8) if mask.dtype == torch.bool else mask
        with torch.cuda.device(q.device):
            rc = spruce_hip.lib().spruce_sparse_prefill_index_amask(
                spruce_hip.ptr(q), spruce_hip.strides(q),
                spruce_hip.ptr(k), spruce_hip.strides(k),
                spruce_hip.ptr(v), spruce_hip.strides(v),
                spruce_hip.ptr(indices), spruce_hip.strides(indices), indices.shape[3],
                spruce_hip.ptr(mview), spruce_hip.strides(mview), mask.shape[1], mask.shape[2], mask.shape[3],
                code, B, Hq, Hkv, T, D, float(scale), spruce_hip.dtype_code(q),
                spruce_hip.variant_code(kernel_variant),
                spruce_hip.ptr(out), out_strides, spruce_hip.stream_of(q))
        spruce_hip.check(rc, "spruce_sparse_prefill_index_amask")
        _record(kernel_variant, Hq, Hkv, D)
        return out
    if key_valid is not None:
        kv8 = _key_valid(key_valid, B, T, q.device)
        zero4 = spruce_hip.strides(torch.empty(0, 0, 0, 0))
        with torch.cuda.device(q.device):
            rc = spruce_hip.lib().spruce_sparse_prefill_index_masked(
                spruce_hip.ptr(q), spruce_hip.strides(q),
                spruce_hip.ptr(k), spruce_hip.strides(k),
                spruce_hip.ptr(v), spruce_hip.strides(v),
                spruce_hip.ptr(indices), spruce_hip.strides(indices), indices.shape[3],
                spruce_hip.ptr(kv8), T, None, zero4, 0, None, None, None,
                spruce_hip.DTYPE_CODES[torch.float32], 0, 1,
                B, Hq, Hkv, T, D, float(scale), spruce_hip.dtype_code(q),
                spruce_hip.variant_code(kernel_variant),
                spruce_hip.ptr(out), out_strides, spruce_hip.stream_of(q))
        spruce_hip.check(rc, "spruce_sparse_prefill_index_masked")
        _record(kernel_variant, Hq, Hkv, D)
        return out
    with torch.cuda.device(q.device):
        rc = spruce_hip.lib().spruce_sparse_prefill_index(
            spruce_hip.ptr(q), spruce_hip.strides(q),
            spruce_hip.ptr(k), spruce_hip.strides(k),
            spruce_hip.ptr(v), spruce_hip.strides(v),
            spruce_hip.ptr(indices), spruce_hip.strides(indices), indices.shape[3],
            B, Hq, Hkv, T, D, float(scale), spruce_hip.dtype_code(q),
            spruce_hip.variant_code(kernel_variant),
            spruce_hip.ptr(out), out_strides, spruce_hip.stream_of(q))
    spruce_hip.check(rc, "spruce_sparse_prefill_index")
    _record(kernel_variant, Hq, Hkv, D)
    return out


def direct_index_sparse_summaries(q, k, v, indices, nodes, table, scale, block_size=64,
                                  kernel_variant="single_head", key_valid=None):
    """Direct-index attention plus residual summaries (sparse/attention.py:226-265).

    indices: int32 ``[B,Hkv,ceil(T/64),K]``; nodes: int32 ``[B,Hkv,ceil(T/64),S]``
    residual tree-node IDs (-1 padding); table: the ``KVSummaryTable`` of
    ``sparse.summaries.build_kv_summary_table`` over the same K/V (keys/values
    ``[B,Hkv,N,P,D]`` float32, log_counts ``[B,N,P]``).  Every listed node adds
    one softmax entry per prototype with a non-empty slice: the summary key's
    score plus log(count), and the summary value.  key_valid: optional bool
    ``[B,T]`` key padding for the exact keys (the table should be built with
    the same token mask).  Returns ``[B,T,Hq,D]``.
    """
    B, Hq, Hkv, T, D = _check_common(q, k, v, block_size, kernel_variant)
    qblocks = (T + block_size - 1) // block_size
    if indices.dim() != 4 or tuple(indices.shape[:3]) != (B, Hkv, qblocks) or indices.dtype != torch.int32:
        raise ValueError("indices must be int32 [B,Hkv,ceil(T/64),K]")
    if nodes.dim() != 4 or tuple(nodes.shape[:3]) != (B, Hkv, qblocks) or nodes.dtype != torch.int32:
        raise ValueError("residual nodes must be int32 [B,Hkv,ceil(T/64),S]")
    keys, values, logc = table.keys, table.values, table.log_counts
    if keys.dim() != 5 or keys.shape[:2] != (B, Hkv) or keys.shape[4] != D or values.shape != keys.shape:
        raise ValueError("summary keys/values must be float32 [B,Hkv,N,P,D]")
    if logc.shape != (B, keys.shape[2], keys.shape[3]):
        raise ValueError("summary log_counts must be [B,N,P]")
    if any(t.dtype != torch.float32 or not t.is_contiguous() for t in (keys, values, logc)):
        raise ValueError("summary tables must be contiguous float32")
    if any(x.stride(-1) != 1 for x in (q, k, v, indices, nodes)):
        raise ValueError("q, k, v, indices and nodes must have a contiguous final dimension")
    if any(t.device != q.device for t in (indices, nodes, keys, values, logc)):
        raise ValueError("indices, nodes and the summary table must be on the same device as q")
    if q.dtype != torch.float32:
        # The kernel rounds the table to the 16-bit input type anyway; a
        # rounded copy (round to nearest even, as the kernel rounds) halves
        # the bytes its producer stages per summary chunk.
        keys, values = keys.to(q.dtype), values.to(q.dtype)
    out, out_strides = _output(q)
    if key_valid is not None:
        kv8 = _key_valid(key_valid, B, T, q.device)
        with torch.cuda.device(q.device):
            rc = spruce_hip.lib().spruce_sparse_prefill_index_masked(
                spruce_hip.ptr(q), spruce_hip.strides(q),
                spruce_hip.ptr(k), spruce_hip.strides(k),
                spruce_hip.ptr(v), spruce_hip.strides(v),
                spruce_hip.ptr(indices), spruce_hip.strides(indices), indices.shape[3],
                spruce_hip.ptr(kv8), T,
                spruce_hip.ptr(nodes), spruce_hip.strides(nodes), nodes.shape[3],
                spruce_hip.ptr(keys), spruce_hip.ptr(values), spruce_hip.ptr(logc),
                spruce_hip.dtype_code(keys), keys.shape[2], keys.shape[3],
                B, Hq, Hkv, T, D, float(scale), spruce_hip.dtype_code(q),
                spruce_hip.variant_code(kernel_variant),
                spruce_hip.ptr(out), out_strides, spruce_hip.stream_of(q))
        spruce_hip.check(rc, "spruce_sparse_prefill_index_masked")
        _record(kernel_variant, Hq, Hkv, D)
        return out
    with torch.cuda.device(q.device):
        rc = spruce_hip.lib().spruce_sparse_prefill_index_summaries(
            spruce_hip.ptr(q), spruce_hip.strides(q),
            spruce_hip.ptr(k), spruce_hip.strides(k),
            spruce_hip.ptr(v), spruce_hip.strides(v),
            spruce_hip.ptr(indices), spruce_hip.strides(indices), indices.shape[3],
            spruce_hip.ptr(nodes), spruce_hip.strides(nodes), nodes.shape[3],
            spruce_hip.ptr(keys), spruce_hip.ptr(values), spruce_hip.ptr(logc),
            spruce_hip.dtype_code(keys), keys.shape[2], keys.shape[3],
            B, Hq, Hkv, T, D, float(scale), spruce_hip.dtype_code(q),
            spruce_hip.variant_code(kernel_variant),
            spruce_hip.ptr(out), out_strides, spruce_hip.stream_of(q))
    spruce_hip.check(rc, "spruce_sparse_prefill_index_summaries")
    _record(kernel_variant, Hq, Hkv, D)
    return out


def direct_index_sparse_csr(q, k, v, indptr, indices, scale, block_size=64,
                            row_order=None, kernel_variant="single_head"):
    """Causal block-sparse attention over variable-length (CSR) block lists.

    Row ``r = (b*Hkv + kv_head)*Qb + query_block`` attends the key blocks
    ``indices[indptr[r]:indptr[r+1]]``.  ``row_order`` (int32 permutation of
    the rows, optional) sets the dispatch order; heaviest rows first balances
    variable row lengths.  Returns ``[B,T,Hq,D]`` in q's dtype.
    """
    B, Hq, Hkv, T, D = _check_common(q, k, v, block_size, kernel_variant)
    qblocks = (T + block_size - 1) // block_size
    rows = B * Hkv * qblocks
    if indptr.dtype != torch.int32 or indices.dtype != torch.int32:
        raise ValueError("indptr and indices must be int32")
    if indptr.dim() != 1 or indptr.numel() != rows + 1:
        raise ValueError(f"indptr must be 1-D with B*Hkv*ceil(T/64)+1 = {rows + 1} entries")
    if not indptr.is_contiguous() or not indices.is_contiguous():
        raise ValueError("indptr and indices must be contiguous")
    if any(x.stride(-1) != 1 for x in (q, k, v)):
        raise ValueError("q, k, and v must have a contiguous final dimension")
    if row_order is not None:
        if row_order.dtype != torch.int32 or row_order.numel() != rows or not row_order.is_contiguous():
            raise ValueError(f"row_order must be a contiguous int32 permutation of {rows} rows")
    for t in (indptr, indices) + ((row_order,) if row_order is not None else ()):
        if t.device != q.device:
            raise ValueError("index tensors must be on the same device as q")
    out, out_strides = _output(q)
    with torch.cuda.device(q.device):
        rc = spruce_hip.lib().spruce_sparse_prefill_csr(
            spruce_hip.ptr(q), spruce_hip.strides(q),
            spruce_hip.ptr(k), spruce_hip.strides(k),
            spruce_hip.ptr(v), spruce_hip.strides(v),
            spruce_hip.ptr(indptr), spruce_hip.ptr(indices), indices.numel(),
            spruce_hip.ptr(row_order),
            B, Hq, Hkv, T, D, float(scale), spruce_hip.dtype_code(q),
            spruce_hip.variant_code(kernel_variant),
            spruce_hip.ptr(out), out_strides, spruce_hip.stream_of(q))
    spruce_hip.check(rc, "spruce_sparse_prefill_csr")
    _record(kernel_variant, Hq, Hkv, D)
    return out


def csr_row_order(indptr, num_kv_heads, batch=1):
    """Dispatch order for the CSR kernel: heaviest rows first, heads interleaved.

    Within each (batch, KV head) the query blocks are sorted by row length,
    longest first (longest processing time first balances the variable
    lengths).  Position ``i`` of the order holds a row of (batch, KV head)
    ``i % (batch*num_kv_heads)``; the kernel deals consecutive positions to the
    8 XCDs, so with ``batch*num_kv_heads`` dividing 8 each XCD's L2 serves one
    KV head's K/V.
    """
    bh = batch * num_kv_heads
    counts = (indptr[1:] - indptr[:-1]).view(bh, -1)
    qblocks = counts.shape[1]
    order = torch.argsort(counts, dim=1, descending=True, stable=True)
    rows = order + torch.arange(bh, device=indptr.device)[:, None] * qblocks
    return rows.t().reshape(-1).to(torch.int32).contiguous()


def kernel_runtime_metadata(kernel_variant):
    """Return the launch configuration of the most recent call of a variant.

    Mirrors kernels/seerattention_direct_index_triton.py:430-447: ``best_config``
    is None until the variant has run once in this process.
    """
    if kernel_variant not in KERNEL_VARIANTS:
        raise ValueError(
            f"kernel_variant must be one of {KERNEL_VARIANTS}, "
            f"got {kernel_variant!r}")
    return {"variant": kernel_variant, "best_config": _LAST_CONFIG.get(kernel_variant)}
