"""CPU oracle for route packing -- TEST INFRASTRUCTURE ONLY.

Only tests/ use this module, as the checker of the HIP packing kernels.

Restatements (numpy, int64 arithmetic, vectorised like the reference):
  pack_mask  selected_mask_to_blocks (scripts/export_selected_blocks.py:37-76):
             local = causal & key >= q - local_window; non-local causal columns
             ranked by a running count and kept while the rank fits
             k_selected - |local|; the kept columns are sentinel-sorted and cut
             to k_selected columns, sentinel -> -1.
  pack_ids   selected_ids_to_blocks (:79-175): IDs valid when 0 <= id < kb,
             id <= q, id < q - local_window and id >= sink (sink clipped to
             kb); sorted, duplicates dropped, kept while the running count of
             distinct IDs fits k_selected - local_count - sink_count; joined
             with the forced sink IDs (s < q - local_window) and the local
             window (q - lw .. q, ids >= 0); sorted and cut to k_selected
             columns, sentinel max(qb, kb) -> -1.

Pinned by tests/test_oracle_packing.py: the reference's own known-answer
cases (tests/test_export_selected_blocks.py:11-101 in the reference), the
mask/IDs equivalence the reference asserts (:83-101), and a per-row
set-based brute force on random inputs.
"""
import numpy as np

PAD_VALUE = -1


def pack_mask(mask, k_selected, local_window=1):
    """mask [L,G,qb,kb] bool -> int32 [1,L,G,qb,min(k_selected, kb)]."""
    mask = np.asarray(mask, dtype=bool)
    if mask.ndim != 4:
        raise ValueError(f"selected_mask must be [L,G,qb,kb], got {tuple(mask.shape)}")
    if k_selected < 1:
        raise ValueError(f"k_selected must be >= 1, got {k_selected}")
    if local_window < 0:
        raise ValueError(f"local_window must be >= 0, got {local_window}")
    if k_selected < local_window + 1:
        raise ValueError(f"k_selected={k_selected} cannot fit local window size {local_window + 1}")
    _, _, qb, kb = mask.shape
    key = np.arange(kb)[None, :]
    qry = np.arange(qb)[:, None]
    causal = key <= qry
    local = (causal & (key >= qry - local_window))[None, None]
    nonlocal_sel = mask & causal[None, None] & ~local
    remaining = k_selected - local.sum(axis=-1)
    rank = np.cumsum(nonlocal_sel, axis=-1)
    keep = local | (nonlocal_sel & (rank <= remaining[..., None]))
    packed = np.sort(np.where(keep, key, kb), axis=-1)[..., :k_selected]
    packed = np.where(packed == kb, PAD_VALUE, packed).astype(np.int32)
    return packed[None]


def pack_ids(ids, k_selected, local_window=1, key_blocks=None, sink_blocks=0):
    """ids [L,G,qb,C] ints -> int32 [1,L,G,qb,W], W = min(k, C + sink + lw + 1)."""
    ids = np.asarray(ids).astype(np.int64)
    if ids.ndim != 4:
        raise ValueError(f"selected_ids must be [L,G,qb,C], got {tuple(ids.shape)}")
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
    L, G, qb, C = ids.shape
    kb = qb if key_blocks is None else int(key_blocks)
    if kb < 1:
        raise ValueError(f"key_blocks must be >= 1, got {kb}")
    sink = min(int(sink_blocks), kb)
    q = np.arange(qb)[None, None, :, None]
    sentinel = max(qb, kb)
    valid = (ids >= 0) & (ids < kb) & (ids <= q) & (ids < q - local_window) & (ids >= sink)
    nl = np.sort(np.where(valid, ids, sentinel), axis=-1)
    unique = nl != sentinel
    if C > 1:
        unique[..., 1:] &= nl[..., 1:] != nl[..., :-1]
    query = np.arange(qb)
    local_count = np.minimum(query + 1, local_window + 1)
    sink_count = np.clip(query - local_window, 0, sink)
    remaining = k_selected - local_count - sink_count
    rank = np.cumsum(unique, axis=-1)
    nl = np.where(unique & (rank <= remaining[None, None, :, None]), nl, sentinel)
    loc = query[:, None] - np.arange(local_window, -1, -1)[None, :]
    loc = np.where(loc >= 0, loc, sentinel)
    snk = np.broadcast_to(np.arange(sink)[None, :], (qb, sink))
    snk = np.where(np.arange(sink)[None, :] < (query[:, None] - local_window), snk, sentinel)
    comb = np.concatenate([nl, np.broadcast_to(snk, (L, G, qb, sink)),
                           np.broadcast_to(loc, (L, G, qb, local_window + 1))], axis=-1)
    packed = np.sort(comb, axis=-1)[..., :k_selected]
    return np.where(packed == sentinel, PAD_VALUE, packed).astype(np.int32)[None]
