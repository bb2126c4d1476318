"""Row-normalised teacher targets and top-k target blocks, on gfx950.

Follows load_teacher's post-processing (selector/targets.py:104-121 in the
reference): mean of the block mass over the query heads of each KV group,
causal mask, ``target = mass / row.clamp_min(eps)``; plus the k blocks with
the largest target per row (selector/loss.py:34-46, selector/recall.py:35),
ordered by target descending with ties to the lower block index and -1
padding where a row has fewer than k causal blocks.
"""
import torch

import spruce_hip


@torch.no_grad()
def teacher_targets(mass, num_kv_heads, k=8, eps=1e-9):
    """mass ``[B, H, Qb, Kb]`` float32 -> dict(target ``[B, G, Qb, Kb]``,
    row_mass ``[B, G, Qb]``, topk int32 ``[B, G, Qb, k]``, cmask ``[Qb, Kb]``)."""
    if not mass.is_cuda:
        raise RuntimeError("teacher_targets (HIP) requires a GPU tensor")
    if mass.dim() != 4 or mass.dtype != torch.float32:
        raise ValueError("mass must be float32 [B, H, Qb, Kb]")
    B, H, Qb, Kb = mass.shape
    G = int(num_kv_heads)
    if G < 1 or H % G:
        raise ValueError(f"H={H} not divisible by G={G}")
    mass = mass.contiguous()
    target = torch.empty((B, G, Qb, Kb), device=mass.device, dtype=torch.float32)
    row_mass = torch.empty((B, G, Qb), device=mass.device, dtype=torch.float32)
    topk = torch.empty((B, G, Qb, k), device=mass.device, dtype=torch.int32)
    with torch.cuda.device(mass.device):
        rc = spruce_hip.lib().spruce_teacher_targets(
            spruce_hip.ptr(mass), B, H, G, Qb, Kb, k, float(eps), spruce_hip.ptr(target),
            spruce_hip.ptr(row_mass), spruce_hip.ptr(topk), spruce_hip.stream_of(mass))
    spruce_hip.check(rc, "spruce_teacher_targets")
    cmask = torch.arange(Kb, device=mass.device)[None, :] <= torch.arange(Qb, device=mass.device)[:, None]
    return {"target": target, "row_mass": row_mass, "topk": topk, "cmask": cmask}


@torch.no_grad()
def teacher_group_mass(mass, num_kv_heads):
    """mass ``[B, H, Qb, Kb]`` float32 -> (group mean with the causal mask
    ``[B, G, Qb, Kb]``, its row sums ``[B, G, Qb]``): the unnormalised half of
    :func:`teacher_targets` (selector/targets.py:104-113)."""
    if not mass.is_cuda:
        raise RuntimeError("teacher_group_mass (HIP) requires a GPU tensor")
    if mass.dim() != 4 or mass.dtype != torch.float32:
        raise ValueError("mass must be float32 [B, H, Qb, Kb]")
    B, H, Qb, Kb = mass.shape
    G = int(num_kv_heads)
    if G < 1 or H % G:
        raise ValueError(f"H={H} not divisible by G={G}")
    mass = mass.contiguous()
    out = torch.empty((B, G, Qb, Kb), device=mass.device, dtype=torch.float32)
    row_mass = torch.empty((B, G, Qb), device=mass.device, dtype=torch.float32)
    with torch.cuda.device(mass.device):
        rc = spruce_hip.lib().spruce_teacher_group_mass(
            spruce_hip.ptr(mass), B, H, G, Qb, Kb, spruce_hip.ptr(out), spruce_hip.ptr(row_mass),
            spruce_hip.stream_of(mass))
    spruce_hip.check(rc, "spruce_teacher_group_mass")
    return out, row_mass


def causal_block_mask(qb, kb, device=None):
    """Query block q may attend key block k iff k <= q (selector/targets.py:54-59)."""
    q = torch.arange(qb, device=device)[:, None]
    kk = torch.arange(kb, device=device)[None, :]
    return kk <= q
