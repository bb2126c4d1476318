"""Reduction of a 4-D decoder mask to key validity for padded-batch prefill
(sparse/attention.py:147-150,173-176,225-229 in the reference), on the CPU:
boolean masks as Transformers' sdpa_mask builds them and additive masks as
the eager path builds them, right and left padding; masks with any other
pattern at a real query position give no key validity (they go to the
kernel as a general mask), and malformed masks raise."""
import pytest
import torch

from sparse.attention import _check_mask_shape, _key_validity


def _sdpa_style(lengths, T, left=False):
    valid = torch.zeros(len(lengths), T, dtype=torch.bool)
    for b, n in enumerate(lengths):
        if left:
            valid[b, T - n:] = True
        else:
            valid[b, :n] = True
    causal = torch.tril(torch.ones(T, T, dtype=torch.bool))
    return (causal[None] & valid[:, None, :])[:, None], valid


@pytest.mark.parametrize("left", [False, True])
def test_bool_and_additive_masks_reduce_to_key_validity(left):
    mask, valid = _sdpa_style([9, 5, 1], 9, left=left)
    assert torch.equal(_key_validity(mask, 3, 9), valid)
    additive = torch.zeros(mask.shape).masked_fill(~mask, torch.finfo(torch.float32).min)
    assert torch.equal(_key_validity(additive, 3, 9), valid)
    inf = torch.zeros(mask.shape).masked_fill(~mask, float("-inf"))
    assert torch.equal(_key_validity(inf.half(), 3, 9), valid)


def test_transformers_sdpa_mask_is_accepted():
    from transformers.masking_utils import sdpa_mask
    am = torch.tensor([[1, 1, 1, 1, 1, 1], [1, 1, 1, 1, 0, 0], [0, 0, 1, 1, 1, 1]]).bool()
    mask = sdpa_mask(batch_size=3, q_length=6, kv_length=6, attention_mask=am)
    assert torch.equal(_key_validity(mask, 3, 6), am)


def test_padding_query_rows_are_not_constrained():
    # Fully unmasked rows at padding query positions (what some mask builders
    # do to keep SDPA from NaN) leave key validity unchanged.
    mask, valid = _sdpa_style([4], 6, left=True)
    mask[0, 0, :2] = True
    assert torch.equal(_key_validity(mask, 1, 6), valid)


def test_fully_masked_padding_rows_are_accepted():
    # Left padding as sdpa_mask builds it: padding query rows attend nothing.
    mask, valid = _sdpa_style([6, 3], 6, left=True)
    assert not mask[1, 0, :3].any()
    assert torch.equal(_key_validity(mask, 2, 6), valid)


@pytest.mark.parametrize("case", ["future_key", "missing_key", "bias", "per_head", "packed",
                                  "padding_row"])
def test_other_mask_patterns_go_to_the_general_mask(case):
    # Not causal key padding: no key validity, the kernel reads the mask itself.
    mask, _ = _sdpa_style([8, 6], 8)
    if case == "future_key":
        mask[0, 0, 3, 5] = True
    elif case == "missing_key":
        mask[1, 0, 4, 2] = False
    elif case == "bias":
        mask = torch.zeros(mask.shape).masked_fill(~mask, -1e9)
        mask[0, 0, 2, 1] = -0.5
    elif case == "per_head":
        mask = mask.expand(2, 2, 8, 8).clone()
        mask[0, 1, 5, 0] = False
    elif case == "packed":
        # Sequences [0, 3) and [3, 8) packed into each row: the last query
        # sees only the second, but the first is not padding.
        seg = torch.tensor([0, 0, 0, 1, 1, 1, 1, 1])
        mask = (torch.tril(torch.ones(8, 8, dtype=torch.bool)) & (seg[:, None] == seg[None, :]))
        mask = mask[None, None].expand(2, 1, 8, 8)
    else:
        # A right-padding query row that attends one padding key.
        mask[1, 0, 7, 6] = True
        mask[1, 0, 7, 0] = False
    _check_mask_shape(mask, 2, 2, 8)
    assert _key_validity(mask, 2, 8) is None


def test_per_head_copies_of_one_padding_mask_reduce_to_key_validity():
    mask, valid = _sdpa_style([8, 6], 8)
    assert torch.equal(_key_validity(mask.expand(2, 4, 8, 8), 2, 8), valid)


@pytest.mark.parametrize("case", ["shape", "dims", "heads", "batch"])
def test_malformed_masks_raise(case):
    mask, _ = _sdpa_style([8, 6], 8)
    if case == "shape":
        mask, match = mask[..., :7], "does not match"
    elif case == "dims":
        mask, match = mask[:, 0], "4D additive"
    elif case == "heads":
        mask, match = mask.expand(2, 3, 8, 8), "1 or 4 heads"
    else:
        mask, match = mask[:1], "does not match"
    with pytest.raises(ValueError, match=match):
        _check_mask_shape(mask, 2, 4, 8)


def test_empty_rows_are_found_per_layer_and_rechecked_after_changes():
    from sparse.attention import _empty_rows
    sel = torch.zeros(2, 3, 2, 4, 2, dtype=torch.int32)        # [B, L, G, Qb, K]
    sel[1, 1, 0, 3] = -1
    sel[0, 1, 1, 2] = -1
    sel[1, 2, 1, 0] = -1
    # The first empty row of each layer in (batch, kv_head, query_block) order.
    assert _empty_rows(sel) == {1: (0, 1, 2), 2: (1, 1, 0)}
    assert _empty_rows(sel) is _empty_rows(sel)                 # one check per tensor
    sel[0, 0, 0, 0] = -1                                        # in place: checked again
    assert _empty_rows(sel) == {0: (0, 0, 0), 1: (0, 1, 2), 2: (1, 1, 0)}
    other = sel.clone()
    other[0, 0, 0, 0] = 5
    assert _empty_rows(other) == {1: (0, 1, 2), 2: (1, 1, 0)}


def test_empty_rows_of_inference_tensors_are_checked_at_every_call():
    # Tensors made under inference_mode (how the reference's scripts run the
    # model) have no version counter: no caching, in-place changes are seen.
    from sparse.attention import _empty_rows
    with torch.inference_mode():
        sel = torch.zeros(1, 2, 1, 3, 2, dtype=torch.int32)
        assert _empty_rows(sel) == {}
        sel[0, 1, 0, 2] = -1
        assert _empty_rows(sel) == {1: (0, 0, 2)}
    assert _empty_rows(sel) == {1: (0, 0, 2)}
