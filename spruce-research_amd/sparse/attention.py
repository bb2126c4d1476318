"""Block-sparse prefill attention entry point for Hugging Face models (HIP).

Drop-in for the reference's sparse/attention.py: ``SPARSE_PREFILL_ATTENTION``,
``sparse_prefill_attention_forward`` with the same signature, validation
messages and exception types (sparse/attention.py:41-81, 83-184, 192-199), and
``register_sparse_prefill_attention``.  The reference computes this with a
host loop of small PyTorch ops; here the whole layer is one launch of the
gfx950 direct-index kernel, which reads ``selected_blocks[:, layer_idx]`` in
place.

With ``residual_summaries=True`` the row's softmax also covers the summary
keys of its residual tree nodes (sparse/attention.py:163-182, 226-265): the
summary table of the layer's K/V is built on the GPU
(``build_kv_summary_table``) and the same kernel appends one key per listed
node and non-empty prototype, scored q.k/sqrt(D) + log(count).

Attention masks (sparse/attention.py:147-150, 173-176, 223-229): a 4-D
decoder mask ``[B, 1 or Hq, T, T]`` -- boolean (True attends, Transformers'
sdpa_mask) or additive (added to the scaled scores) -- takes one of two
kernels.  When it is exactly "causal and key is a real token" at every real
query position (padded batches), it is reduced to per-token key validity,
which the kernel applies to every listed key block and which the residual
summary table excludes.  Any other mask (block-diagonal packed sequences,
score biases, per-head masks) is read by the kernel itself and added to the
score of every listed causal key, as the reference adds its slice.  Outputs
at query positions with no surviving key are not defined (the kernel writes
zeros; the reference's softmax gives NaN there).

Differences, all raising instead of computing something else:
  * ``block_size`` must be 64 and ``head_dim`` 64 or 128 (the kernel's tile);
  * residual summaries with a mask other than causal key padding.
A boolean mask attends where True (Transformers' convention); the reference
adds a boolean mask's 0/1 values to the scores like a float mask.
"""
import math
import weakref
from typing import Optional

import torch

from interfaces.residual_summaries import (build_residual_tree_layout,
                                          validate_residual_summary_nodes)
from interfaces.validator import validate_selected_blocks
from kernels.direct_index import direct_index_sparse_prefill, direct_index_sparse_summaries
from sparse.config import SUMMARY_MODES, SUMMARY_PROTOTYPES
from sparse.summaries import build_kv_summary_table, token_validity_from_attention_mask  # noqa: F401

SPARSE_PREFILL_ATTENTION = "spruce_sparse_prefill"


def _layer_index(module: torch.nn.Module) -> int:
    for name in ("layer_idx", "layer_id"):
        value = getattr(module, name, None)
        if value is not None:
            return int(value)
    raise ValueError(
        "Sparse prefill attention needs module.layer_idx (or module.layer_id) "
        "to select the correct selected_blocks layer."
    )


def _validate_inputs(query, key, value, selected_blocks, block_size, layer_idx, validate_blocks):
    """Shape checks of sparse/attention.py:41-81, same messages."""
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise ValueError("query, key, and value must be [batch, heads, tokens, head_dim]")
    if key.shape != value.shape:
        raise ValueError(f"key/value shape mismatch: {tuple(key.shape)} vs {tuple(value.shape)}")
    if query.shape[0] != key.shape[0] or query.shape[-1] != key.shape[-1]:
        raise ValueError("query and key must have the same batch size and head dimension")
    if query.shape[-2] != key.shape[-2]:
        raise ValueError(
            "Stage 3.2 is prefill-only: query and key lengths must match "
            f"(got {query.shape[-2]} and {key.shape[-2]})."
        )
    if block_size < 1:
        raise ValueError(f"block_size must be positive, got {block_size}")
    if query.shape[1] % key.shape[1]:
        raise ValueError(
            f"query heads ({query.shape[1]}) must be divisible by KV heads ({key.shape[1]})")
    if validate_blocks:
        validate_selected_blocks(selected_blocks)
    batch, layers, groups, query_blocks, _ = selected_blocks.shape
    expected_blocks = math.ceil(query.shape[-2] / block_size)
    if batch != query.shape[0] or layers <= layer_idx:
        raise ValueError(
            f"selected_blocks shape {tuple(selected_blocks.shape)} does not cover "
            f"batch {query.shape[0]} and layer {layer_idx}")
    if groups != key.shape[1]:
        raise ValueError(
            f"selected_blocks has {groups} KV groups, model has {key.shape[1]} KV heads")
    if query_blocks != expected_blocks:
        raise ValueError(
            f"selected_blocks has {query_blocks} query blocks; expected {expected_blocks} "
            f"for seq_len={query.shape[-2]} and block_size={block_size}")


_EMPTY_ROWS = [None]   # (weakref to selected_blocks, its version, {layer: first empty row})


def _empty_rows(selected_blocks: torch.Tensor) -> dict:
    """{layer: (batch, kv_head, query_block) of its first row with no listed
    block}, for every layer of ``selected_blocks`` at once.  Reading the
    answer back waits for the GPU, so it is done once per selected_blocks
    tensor (the model's layers share one) and kept while the tensor is alive
    and unmodified, instead of stalling the host at every layer.  Tensors
    made under ``torch.inference_mode`` have no version counter, so an
    in-place change to them could not be seen: they are checked at every
    call."""
    tracked = not selected_blocks.is_inference()
    last = _EMPTY_ROWS[0]
    if (tracked and last is not None and last[0]() is selected_blocks
            and last[1] == selected_blocks._version):
        return last[2]
    empty = ~(selected_blocks >= 0).any(dim=-1)        # [B, L, G, Qb]
    found = {}
    if bool(empty.any()):
        for b, layer, g, qb in torch.nonzero(empty).tolist():
            found.setdefault(layer, (b, g, qb))
    if tracked:
        _EMPTY_ROWS[0] = (weakref.ref(selected_blocks), selected_blocks._version, found)
    return found


def _check_mask_shape(attention_mask: torch.Tensor, batch: int, heads: int, seq_len: int) -> None:
    if attention_mask.dim() != 4:
        raise ValueError(
            "Sparse prefill expects the Transformers 4D additive attention mask; "
            f"got shape {tuple(attention_mask.shape)}")
    if attention_mask.shape[0] != batch or tuple(attention_mask.shape[-2:]) != (seq_len, seq_len):
        raise ValueError(
            f"attention mask {tuple(attention_mask.shape)} does not match batch {batch} and "
            f"{seq_len} query/key tokens")
    if attention_mask.shape[1] not in (1, heads):
        raise ValueError(
            f"attention mask {tuple(attention_mask.shape)} must have 1 or {heads} heads")


def _key_validity(attention_mask: torch.Tensor, batch: int, seq_len: int) -> Optional[torch.Tensor]:
    """Key validity ``[batch, seq_len]`` bool when the 4-D decoder mask is
    causal key padding (the same for every head, 0 / -inf or finfo.min
    values, or bool); None for any other mask, which then goes to the kernel
    as a general additive mask.

    A key is real when the last query position attends it: in a causal
    decoder mask that row sees every real key, with left or right padding,
    and it is never a fully masked padding row that a mask builder may have
    opened up to keep SDPA from producing NaN.  Every real query row must be
    causal over the real keys; a padding query row may also attend nothing
    or everything (Transformers opens fully masked rows up), but nothing
    else, so packed sequences (a block-diagonal mask) are not taken for
    left padding."""
    m = attention_mask
    if m.shape[1] != 1 and not bool((m == m[:, :1]).all()):
        return None
    m = m[:, 0]
    if m.dtype == torch.bool:
        attend = m
    else:
        attend = m >= 0
        if bool((m[attend] != 0).any()) or bool((m[~attend] > torch.finfo(m.dtype).min / 2).any()):
            return None
    valid = attend[:, -1, :]
    keys = torch.arange(seq_len, device=m.device)
    for r0 in range(0, seq_len, 2048):
        r1 = min(r0 + 2048, seq_len)
        rows = attend[:, r0:r1]
        expected = (keys[None, :] <= keys[r0:r1, None])[None] & valid[:, None, :]
        differs = (rows != expected).any(dim=-1)
        opened = rows.all(dim=-1) | ~rows.any(dim=-1)
        if bool((differs & (valid[:, r0:r1] | ~opened)).any()):
            return None
    return valid


def sparse_prefill_attention_forward(
    module: torch.nn.Module,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: Optional[torch.Tensor],
    *,
    selected_blocks: torch.Tensor,
    block_size: int,
    validate_selected_blocks_input: bool = True,
    residual_summaries: bool = False,
    residual_summary_nodes: Optional[torch.Tensor] = None,
    summary_prototypes: int = 1,
    summary_mode: str = "mean",
    summary_checkpoint: Optional[str] = None,
    validate_residual_summary_nodes_input: bool = True,
    **kwargs,
) -> tuple[torch.Tensor, None]:
    """Transformers AttentionInterface implementation for sparse prefill.

    query ``[B,Hq,T,D]``, key/value ``[B,Hkv,T,D]``, ``selected_blocks``
    ``[B,L,Hkv,ceil(T/block_size),K]`` int32.  Returns ``([B,T,Hq,D], None)``.
    """
    del kwargs
    layer_idx = _layer_index(module)
    _validate_inputs(query, key, value, selected_blocks, block_size, layer_idx,
                     validate_blocks=validate_selected_blocks_input)
    if summary_prototypes not in SUMMARY_PROTOTYPES:
        raise ValueError(
            f"summary_prototypes must be one of {SUMMARY_PROTOTYPES}, got {summary_prototypes}")
    if summary_mode not in SUMMARY_MODES:
        raise ValueError(f"summary_mode must be one of {SUMMARY_MODES}, got {summary_mode!r}")
    if residual_summaries:
        if residual_summary_nodes is None:
            raise ValueError(
                "residual_summaries=True requires residual_summary_nodes; "
                "construct the complete frontier before model forward")
        if summary_mode == "learned":
            if not summary_checkpoint:
                raise ValueError("summary_mode='learned' requires summary_checkpoint")
            raise NotImplementedError(
                "The learned compressor is gated on deterministic-summary "
                "evaluation and is not implemented before that gate passes.")
        if validate_residual_summary_nodes_input:
            validate_residual_summary_nodes(
                selected_blocks, residual_summary_nodes,
                validate_selected=not validate_selected_blocks_input)
    key_valid = None
    general_mask = None
    if attention_mask is not None:
        _check_mask_shape(attention_mask, query.shape[0], query.shape[1], query.shape[-2])
        key_valid = _key_validity(attention_mask, query.shape[0], query.shape[-2])
        if key_valid is None:
            if residual_summaries:
                raise ValueError(
                    "residual summaries on the HIP sparse-prefill path need a causal key-padding "
                    "attention mask; this mask has another pattern")
            general_mask = attention_mask   # added to the scores inside the kernel
        elif bool(key_valid.all()):
            key_valid = None      # no padding: the plain kernel
    if block_size != 64:
        raise ValueError("the HIP sparse-prefill kernel requires block_size=64")
    indices = selected_blocks[:, layer_idx].to(device=query.device, dtype=torch.int32).contiguous()
    # The reference raises on a row with no selected block (sparse/attention.py:192-199).
    empty_row = _empty_rows(selected_blocks).get(layer_idx)
    if empty_row is not None:
        b, g, qb = empty_row
        raise ValueError(
            "selected_blocks leaves an attention row empty at "
            f"batch={b}, layer={layer_idx}, kv_head={g}, query_block={qb}")
    D = query.shape[-1]
    if not residual_summaries:
        output = direct_index_sparse_prefill(
            query, key, value, indices, scale=1.0 / math.sqrt(D), block_size=block_size,
            key_valid=key_valid, attn_mask=general_mask)
        return output, None
    # Residual summaries (sparse/attention.py:163-182): the frontier nodes of
    # this layer, and the summary table of this layer's K/V over the tree.
    if residual_summary_nodes.shape[:4] != selected_blocks.shape[:4]:
        raise ValueError(
            "residual_summary_nodes must match selected_blocks through the query-block dimension")
    nodes = residual_summary_nodes[:, layer_idx].to(device=query.device, dtype=torch.int32).contiguous()
    layout = build_residual_tree_layout(indices.shape[2])
    table = build_kv_summary_table(key, value, layout, block_size=block_size,
                                   prototypes=summary_prototypes, token_mask=key_valid)
    output = direct_index_sparse_summaries(
        query, key, value, indices, nodes, table, scale=1.0 / math.sqrt(D), block_size=block_size,
        key_valid=key_valid)
    return output, None


def register_sparse_prefill_attention(name: str = SPARSE_PREFILL_ATTENTION) -> str:
    """Register this backend with Transformers (sparse/attention.py:277-292).

    The mask formatter is Transformers' sdpa_mask, as in the reference: no
    mask for unpadded causal prefill, a boolean [B, 1, T, T] mask for padded
    batches (reduced to key validity here).
    """
    try:
        from transformers import AttentionInterface, AttentionMaskInterface
        from transformers.masking_utils import sdpa_mask
    except ImportError as error:
        raise RuntimeError("register_sparse_prefill_attention requires transformers") from error
    AttentionInterface.register(name, sparse_prefill_attention_forward)
    AttentionMaskInterface.register(name, sdpa_mask)
    return name
