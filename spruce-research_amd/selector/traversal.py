"""Top-down beam traversal of the key tree on gfx950
(scripts/eval_tree_traversal.py:43-132 in the reference).

``traverse_to_leaf_ids(gate, q_feat, key_levels, beam, radix=2,
layer_chunk=1)`` returns compact leaf IDs ``[L,G,qb,C]`` as the reference
does: from the root, each level scores only the children of the current beam
(MaxSim of the gate's projected prototypes), drops children past the level's
last node or starting after the query block, and keeps the best
``min(beam, candidates, level nodes)``, score-descending, ``-1`` where no
valid candidate was left.  The query and every tree node are projected once;
the walk itself is one HIP launch (``spruce_tree_traverse``, one wavefront per
query row), so no ``[.., C, P, p]`` candidate tensor is ever gathered.
``layer_chunk`` is accepted for signature compatibility; nothing is chunked.

Equal scores go to the lower node (the reference leaves tie order to
``torch.topk``).  The reference's module name ``scripts.eval_tree_traversal``
re-exports these functions.
"""
import math

import torch

import spruce_hip


def child_parent_index(parent_level, child_level):
    """Map each child node to its parent node in the next coarser level."""
    parent_for_child = torch.searchsorted(parent_level.ends, child_level.starts, right=True)
    if torch.any(parent_for_child >= parent_level.ends.numel()):
        raise ValueError("a child range falls outside all parent ranges")
    parent_starts = parent_level.starts.index_select(0, parent_for_child)
    parent_ends = parent_level.ends.index_select(0, parent_for_child)
    valid = (parent_starts <= child_level.starts) & (child_level.ends <= parent_ends)
    if not bool(valid.all()):
        raise ValueError("a child range does not fit exactly one parent range")
    return parent_for_child


def output_width(num_leaves, radix, beam):
    """Width C of the traversal output: the beam width after the leaf level."""
    counts = [num_leaves]
    while counts[-1] > 1:
        counts.append((counts[-1] + radix - 1) // radix)
    width = 1
    for n in reversed(counts[:-1]):
        width = min(beam, width * radix, n)
    return width


def traverse_projected(projected_q, projected_k_all, num_leaves, beam, radix, div, rows_kernel=False):
    """Raw form: projected_q [L,G,qb,Pq,p], projected_k_all [L,G,N,Pk,p]
    (every node, leaf-first IDs) or the interleaved [L,G,N,p/4,Pk,4] of
    ``FlatGate.project_key_levels(..., interleaved=True)``, float32 ->
    [L,G,qb,C] int64 leaf IDs (the same for both layouts).  A rows-layout
    table is copied into the interleaved layout first (the walk reads it
    about twice as fast, which pays for the copy), unless ``rows_kernel``
    asks for the kernel that reads the rows layout in place."""
    L, G, qb, Pq, p = projected_q.shape
    interleaved = projected_k_all.dim() == 6
    if interleaved:
        N, Pk = projected_k_all.shape[2], projected_k_all.shape[4]
        ok = projected_k_all.shape[3] * 4 == p and projected_k_all.shape[5] == 4
    else:
        N, Pk = projected_k_all.shape[2], projected_k_all.shape[3]
        ok = projected_k_all.dim() == 5 and projected_k_all.shape[4] == p
    if projected_k_all.shape[:2] != (L, G) or not ok:
        raise ValueError("projected query and key shapes disagree")
    if not interleaved and not rows_kernel and p % 4 == 0:
        projected_k_all = projected_k_all.reshape(L, G, N, Pk, p // 4, 4).transpose(3, 4)
        interleaved = True
    qp = projected_q.float().contiguous()
    kp = projected_k_all.float().contiguous()
    C = output_width(num_leaves, radix, beam)
    out = torch.empty((L, G, qb, C), device=qp.device, dtype=torch.int32)
    with torch.cuda.device(qp.device):
        rc = spruce_hip.lib().spruce_tree_traverse(
            spruce_hip.ptr(qp), spruce_hip.ptr(kp), L * G, qb, num_leaves, Pq, Pk, p, radix, beam,
            float(div), spruce_hip.ptr(out), C, 1 if interleaved else 0, spruce_hip.stream_of(qp))
    spruce_hip.check(rc, "spruce_tree_traverse")
    return out.long()


@torch.no_grad()
def traverse_to_leaf_ids(gate, q_feat, key_levels, beam, radix=2, layer_chunk=1):
    """Compact selected leaf IDs ``[L,G,qb,C]`` (int64); invalid slots are -1."""
    if beam < 1:
        raise ValueError(f"beam must be >= 1, got {beam}")
    if radix < 2:
        raise ValueError(f"radix must be >= 2, got {radix}")
    if layer_chunk < 1:
        raise ValueError(f"layer_chunk must be >= 1, got {layer_chunk}")
    root_level = key_levels[-1]
    if root_level.features.shape[2] != 1:
        raise ValueError("key tree must end in exactly one root node")
    kb = key_levels[0].features.shape[2]
    for below, above in zip(key_levels, key_levels[1:]):
        if above.features.shape[2] != (below.features.shape[2] + radix - 1) // radix:
            raise ValueError("key tree levels do not match the radix")
    if not q_feat.is_cuda:
        raise RuntimeError("traverse_to_leaf_ids (HIP) requires GPU tensors")
    projected_q = gate.project_queries(q_feat)
    if hasattr(gate, "project_key_levels"):
        projected_k = gate.project_key_levels([lvl.features for lvl in key_levels], interleaved=True)
    else:
        projected_k = gate.project_keys(torch.cat([lvl.features for lvl in key_levels], dim=2))
    return traverse_projected(projected_q, projected_k, kb, beam, radix, math.sqrt(gate.proj_dim))


@torch.no_grad()
def leaf_ids_to_mask(selected_ids, leaf_count):
    """Convert compact ``[L,G,qb,C]`` IDs to an evaluation-only leaf mask."""
    if selected_ids.dim() != 4:
        raise ValueError(f"selected_ids must be [L,G,qb,C], got {tuple(selected_ids.shape)}")
    if leaf_count < 1:
        raise ValueError(f"leaf_count must be >= 1, got {leaf_count}")
    L, G, qb = selected_ids.shape[:3]
    safe = selected_ids.clamp(min=0, max=leaf_count).masked_fill(selected_ids < 0, leaf_count)
    with_pad = torch.zeros((L, G, qb, leaf_count + 1), dtype=torch.bool, device=selected_ids.device)
    with_pad.scatter_(-1, safe, True)
    return with_pad[..., :leaf_count]


@torch.no_grad()
def traverse_to_leaf(gate, q_feat, key_levels, beam, radix=2, layer_chunk=1):
    """Evaluation mask ``[L,G,qb,kb]`` from the compact traversal."""
    ids = traverse_to_leaf_ids(gate, q_feat, key_levels, beam, radix=radix, layer_chunk=layer_chunk)
    return leaf_ids_to_mask(ids, key_levels[0].features.shape[2])
