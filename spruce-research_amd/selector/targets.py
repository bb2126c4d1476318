"""Teacher artifacts -> selector inputs and targets (selector/targets.py:1-123 in the reference).

A teacher file holds, for one document: ``pooled [1, L, H, qb, kb]`` block
mass per query head, ``pooledQ [1, L, G, qb, P, d]`` / ``pooledK
[1, L, G, kb, P, d]`` prototype features, ``proto`` (P), ``seq_len``,
``block_size`` and optional metadata.  The functions here keep the
reference's names, arguments, return keys and error messages.

Differences from the reference:
* files are read with ``torch.load(..., weights_only=True)``: tensors,
  numbers, strings, lists and dicts load, pickled objects are refused;
* the target post-processing (group mean over each KV group's query heads,
  causal mask, row normalisation) runs in the HIP kernels of
  ``teacher.targets`` on a GPU, whatever ``device`` the results go to; with no
  GPU it raises ``RuntimeError`` (there is no CPU path).
"""
import torch

from teacher.targets import causal_block_mask, teacher_group_mass, teacher_targets

__all__ = ["load_selector_features", "causal_block_mask", "load_teacher"]

_NO_PROTO = ("{path} lacks P-prototype selector features ('proto' key / 6-D pooledK). "
             "It predates multi-prototype extraction. Re-extract with "
             "scripts/extract_teacher_targets.py to regenerate it.")


def _read(path):
    return torch.load(path, map_location="cpu", weights_only=True)


def _has_proto(d):
    return d.get("proto") is not None and d["pooledK"].dim() == 6


def _meta(d, L, G, qb, kb, head_dim):
    return {
        "seq_len": int(d["seq_len"]), "block_size": int(d["block_size"]),
        "requested_length": int(d.get("requested_length", d["seq_len"])),
        "needle_block": int(d.get("needle_block", -1)),
        "num_layers": L, "num_groups": G, "qb": qb, "kb": kb,
        "head_dim": head_dim, "proto": int(d["proto"]),
    }


def load_selector_features(path, device="cpu"):
    """Only the pooled Q/K prototype features (selector/targets.py:21-51): the
    file is read on the host and just ``q_feat``/``k_feat`` move to ``device``."""
    d = _read(path)
    if not _has_proto(d):
        raise KeyError(
            f"{path} lacks P-prototype selector features ('proto' key / 6-D pooledK). "
            "Re-extract with scripts/extract_teacher_targets.py to regenerate it.")
    q_feat = d["pooledQ"].float()[0].to(device)
    k_feat = d["pooledK"].float()[0].to(device)
    L, G, qb, _, head_dim = q_feat.shape
    meta = _meta(d, L, G, qb, k_feat.shape[2], head_dim)
    meta.update({
        "rope": d.get("rope"),
        "features_only": bool(d.get("features_only", False)),
        "prompt_format": d.get("prompt_format"),
        "dense_screen_accepted": bool(d.get("dense_screen", {}).get("accepted", False)),
        "case_id": d.get("case_id"),
        "depth": d.get("depth"),
    })
    return {"q_feat": q_feat, "k_feat": k_feat, "meta": meta}


def _compute_device(device):
    dev = torch.device(device)
    if dev.type == "cuda":
        return dev
    if not torch.cuda.is_available():
        raise RuntimeError("load_teacher post-processes the teacher mass with HIP kernels and needs a GPU")
    return torch.device("cuda", torch.cuda.current_device())


def load_teacher(path, device="cpu", eps=1e-9, defer_normalization=False):
    """Selector training tensors from a teacher file (selector/targets.py:62-123).

    Returns ``q_feat [L, G, qb, P, d]``, ``k_feat [L, G, kb, P, d]``,
    ``cmask [qb, kb]`` and ``meta``, plus either ``target [L, G, qb, kb]``
    (group-mean mass, causal, each row divided by max(row sum, eps)) and
    ``row_mass [L, G, qb]``, or with ``defer_normalization`` the unnormalised
    ``mass`` in the features' stored dtype and ``normalization_eps``."""
    d = _read(path)
    if not _has_proto(d):
        raise KeyError(_NO_PROTO.format(path=path))
    if d.get("pooled") is None:
        raise ValueError(
            f"{path} is a selector-feature-only artifact and has no dense "
            "teacher mass; it can be used for traversal/128K replay but not training")
    stored_dtype = d["pooledQ"].dtype
    q_feat = d["pooledQ"][0] if defer_normalization else d["pooledQ"].float()[0]
    k_feat = d["pooledK"][0] if defer_normalization else d["pooledK"].float()[0]
    pooled = d["pooled"][0]                                   # [L, H, qb, kb]
    L, H, qb, kb = pooled.shape
    G = k_feat.shape[1]
    if H % G:
        raise AssertionError(f"H={H} not divisible by G={G}")
    meta = _meta(d, L, G, qb, kb, q_feat.shape[-1])
    meta.update({
        "prompt_format": d.get("prompt_format"),
        "dense_screen_accepted": bool(d.get("dense_screen", {}).get("accepted", False)),
        "case_id": d.get("case_id"),
        "depth": d.get("depth"),
    })
    work = _compute_device(device)
    mass = pooled.to(device=work, dtype=torch.float32).contiguous()
    cmask = causal_block_mask(qb, kb, device=device)
    q_feat, k_feat = q_feat.to(device), k_feat.to(device)
    if defer_normalization:
        group_mass, _ = teacher_group_mass(mass, G)
        return {"q_feat": q_feat, "k_feat": k_feat, "mass": group_mass.to(device=device, dtype=stored_dtype),
                "cmask": cmask, "meta": meta, "normalization_eps": float(eps)}
    t = teacher_targets(mass, G, k=1, eps=eps)
    return {"q_feat": q_feat, "k_feat": k_feat, "target": t["target"].to(device), "cmask": cmask,
            "row_mass": t["row_mass"].to(device), "meta": meta}
