"""Reduction of a 4-D decoder mask to key validity for padded-batch prefill
(sparse/attention.py:147-150,173-176,225-229 in the reference), on the CPU:
boolean masks as Transformers' sdpa_mask builds them and additive masks as
the eager path builds them, right and left padding; masks with any other
pattern at a real query position are rejected."""
import pytest
import torch

from sparse.attention import _key_validity


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


@pytest.mark.parametrize("case", ["future_key", "missing_key", "bias", "per_head", "shape", "dims"])
def test_other_mask_patterns_raise(case):
    mask, _ = _sdpa_style([8, 6], 8)
    if case == "future_key":
        mask[0, 0, 3, 5] = True
        match = "another pattern"
    elif case == "missing_key":
        mask[1, 0, 4, 2] = False
        match = "another pattern"
    elif case == "bias":
        mask = torch.zeros(mask.shape).masked_fill(~mask, -1e9)
        mask[0, 0, 2, 1] = -0.5
        match = "score biases"
    elif case == "per_head":
        mask = mask.expand(2, 2, 8, 8).clone()
        mask[0, 1, 5, 0] = False
        match = "per-head"
    elif case == "shape":
        mask = mask[..., :7]
        match = "does not match"
    else:
        mask = mask[:, 0]
        match = "4D additive"
    with pytest.raises(ValueError, match=match):
        _key_validity(mask, 2, 8)
