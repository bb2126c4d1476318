"""Route packing into the selected_blocks contract, on gfx950.

Same names, arguments, policies and errors as the reference's
``selected_mask_to_blocks`` and ``selected_ids_to_blocks``
(scripts/export_selected_blocks.py:37-175).  One HIP kernel per call
(``spruce_pack_selected_mask`` / ``spruce_pack_selected_ids``); rows come out
int32, ascending, padded with PAD_VALUE, shaped ``[1, L, G, qb, W]``.
"""
import torch

import spruce_hip
from interfaces.validator import PAD_VALUE

__all__ = ["PAD_VALUE", "selected_mask_to_blocks", "selected_ids_to_blocks"]


def _device_tensor(t, name):
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (HIP route packing)")


@torch.no_grad()
def selected_mask_to_blocks(selected_mask, k_selected, local_window=1):
    """[L,G,qb,kb] bool mask -> selected_blocks int32 [1,L,G,qb,min(K, kb)].

    The local blocks q-local_window..q are forced first, then the lowest
    selected causal non-local blocks fill the row up to k_selected.
    """
    if selected_mask.dim() != 4:
        raise ValueError(f"selected_mask must be [L,G,qb,kb], got {tuple(selected_mask.shape)}")
    if k_selected < 1:
        raise ValueError(f"k_selected must be >= 1, got {k_selected}")
    if local_window < 0:
        raise ValueError(f"local_window must be >= 0, got {local_window}")
    if k_selected < local_window + 1:
        raise ValueError(
            f"k_selected={k_selected} cannot fit local window size {local_window + 1}")
    _device_tensor(selected_mask, "selected_mask")
    L, G, qb, kb = selected_mask.shape
    mask = selected_mask
    if mask.dtype != torch.bool:
        mask = mask != 0
    mask = mask.contiguous().view(torch.uint8)
    width = min(int(k_selected), kb)
    out = torch.empty((1, L, G, qb, width), device=mask.device, dtype=torch.int32)
    if out.numel() == 0:
        return out
    with torch.cuda.device(mask.device):
        rc = spruce_hip.lib().spruce_pack_selected_mask(
            mask.data_ptr(), L * G * qb, qb, kb, int(k_selected), int(local_window),
            out.data_ptr(), width, spruce_hip.stream_of(mask))
    spruce_hip.check(rc, "spruce_pack_selected_mask")
    return out


@torch.no_grad()
def selected_ids_to_blocks(selected_ids, k_selected, local_window=1, key_blocks=None, sink_blocks=0):
    """Pack compact traversal IDs ``[L,G,qb,C]`` into selected_blocks.

    Forced sink blocks (the first ``sink_blocks`` key blocks, where they sit
    before the local window) and the local window take priority; the smallest
    distinct causal non-local IDs fill the remaining slots.  Output width is
    ``min(k_selected, C + min(sink_blocks, key_blocks) + local_window + 1)``.
    """
    if selected_ids.dim() != 4:
        raise ValueError(f"selected_ids must be [L,G,qb,C], got {tuple(selected_ids.shape)}")
    if k_selected < 1:
        raise ValueError(f"k_selected must be >= 1, got {k_selected}")
    if local_window < 0:
        raise ValueError(f"local_window must be >= 0, got {local_window}")
    if sink_blocks < 0:
        raise ValueError(f"sink_blocks must be >= 0, got {sink_blocks}")
    if k_selected < local_window + 1 + sink_blocks:
        raise ValueError(
            f"k_selected={k_selected} cannot fit local window size "
            f"{local_window + 1} plus {sink_blocks} sink block(s)")
    L, G, qb, C = selected_ids.shape
    kb = qb if key_blocks is None else int(key_blocks)
    if kb < 1:
        raise ValueError(f"key_blocks must be >= 1, got {kb}")
    _device_tensor(selected_ids, "selected_ids")
    ids = selected_ids
    if ids.dtype not in (torch.int32, torch.int64):
        ids = ids.to(torch.int64)
    ids = ids.contiguous()
    sink = min(int(sink_blocks), kb)
    width = min(int(k_selected), C + sink + int(local_window) + 1)
    out = torch.empty((1, L, G, qb, width), device=ids.device, dtype=torch.int32)
    if out.numel() == 0:
        return out
    with torch.cuda.device(ids.device):
        rc = spruce_hip.lib().spruce_pack_selected_ids(
            ids.data_ptr(), ids.element_size(), L * G * qb, qb, C, kb, int(k_selected),
            int(local_window), int(sink_blocks), out.data_ptr(), width, spruce_hip.stream_of(ids))
    spruce_hip.check(rc, "spruce_pack_selected_ids")
    return out
