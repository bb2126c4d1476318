"""The ``selected_blocks`` contract check (interfaces/validator.py:7-62).

Rules per row ``t[b, l, g, q, :]`` (interfaces/selected_blocks_spec.md:1-20):
causal (every real ID <= q), sorted, no duplicates, the local window
``max(0, q - local_window) .. q`` present, and PAD_VALUE (-1) only as trailing
padding.  The reference walks the rows in Python; this version evaluates every
rule for every row with tensor ops (on the tensor's own device) and then
reports the first violating row in (b, l, g, q) order with the first failing
rule in the reference's rule order, raising ``AssertionError`` with the same
message text.
"""
import torch

PAD_VALUE = -1
LOCAL_WINDOW = 1


def _row_violations(t, local_window):
    """Bool [rows, 5] -- causal, sorted, duplicate, local window, padding."""
    batch, layer, group, qblocks, k = t.shape
    rows = t.reshape(-1, k).to(torch.long)
    q = torch.arange(qblocks, device=t.device).repeat(batch * layer * group)[:, None]
    real = rows != PAD_VALUE

    causal = (real & (rows > q)).any(dim=-1)

    # Compact the real IDs to the front (stable), keeping their row order.
    order = torch.argsort((~real).to(torch.int8), dim=-1, stable=True)
    packed = rows.gather(-1, order)
    n_real = real.sum(dim=-1, keepdim=True)
    pos = torch.arange(k, device=t.device)[None, :]
    pair = pos[:, 1:] < n_real  # both packed[i] and packed[i+1] are real
    unsorted = ((packed[:, 1:] < packed[:, :-1]) & pair).any(dim=-1)
    duplicate = ((packed[:, 1:] == packed[:, :-1]) & pair).any(dim=-1)

    # Every block in max(0, q - w) .. q must appear among the real IDs.
    offsets = torch.arange(local_window + 1, device=t.device)[None, :]
    required = q - offsets  # [rows, w+1]
    needed = required >= 0
    present = (rows[:, None, :] == required[:, :, None]) & real[:, None, :]
    missing_local = (needed & ~present.any(dim=-1)).any(dim=-1)

    # Padding must be trailing: no real ID after the first PAD.
    seen_pad = (~real).to(torch.int32).cumsum(dim=-1) > 0
    bad_pad = (seen_pad & real).any(dim=-1)
    return torch.stack([causal, unsorted, duplicate, missing_local, bad_pad], dim=-1)


def validate_selected_blocks(t: torch.Tensor, local_window: int = LOCAL_WINDOW) -> None:
    """Raise AssertionError at the first contract violation of ``t``.

    Shape: ``[batch, layer, kv_head_group, query_block, K_selected_blocks]``.
    """
    assert t.dim() == 5, (
        f"Expected 5D tensor [batch, layer, kv_head_group, query_block, "
        f"K_selected_blocks], got {t.dim()}D with shape {tuple(t.shape)}"
    )
    assert t.dtype == torch.int32, f"Expected int32, got {t.dtype}"
    assert local_window >= 0, f"local_window must be >= 0, got {local_window}"
    batch, layer, group, qblocks, k = t.shape
    if t.numel() == 0:
        if k == 0 and qblocks > 0 and batch * layer * group > 0:
            # A zero-width row cannot hold the local window.
            assert False, (
                f"Missing local-window block(s) at [b=0, l=0, g=0, q=0]: "
                f"missing [0], row=[]")
        return
    bad = _row_violations(t, local_window)
    any_bad = bad.any(dim=-1)
    if not bool(any_bad.any()):
        return
    first = int(torch.nonzero(any_bad)[0, 0])
    rule = int(torch.nonzero(bad[first])[0, 0])
    q = first % qblocks
    g = (first // qblocks) % group
    l = (first // (qblocks * group)) % layer
    b = first // (qblocks * group * layer)
    row = t[b, l, g, q].tolist()
    real_ids = [x for x in row if x != PAD_VALUE]
    where = f"[b={b}, l={l}, g={g}, q={q}]"
    if rule == 0:
        block_id = next(x for x in real_ids if x > q)
        raise AssertionError(
            f"Causal violation at {where}: block {block_id} is in the future (q={q})")
    if rule == 1:
        raise AssertionError(f"Not sorted at {where}: {real_ids}")
    if rule == 2:
        raise AssertionError(f"Duplicate block IDs at {where}: {real_ids}")
    if rule == 3:
        required = list(range(max(0, q - local_window), q + 1))
        missing = [x for x in required if x not in real_ids]
        raise AssertionError(
            f"Missing local-window block(s) at {where}: missing {missing}, row={real_ids}")
    raise AssertionError(f"Padding is not trailing-only at {where}: {row}")
