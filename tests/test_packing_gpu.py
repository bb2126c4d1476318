"""Route packing kernels (HIP, through the C ABI) against the oracle.

Bar: bit-exact int32 rows.  Cases cover the reference's known answers
(tests/test_export_selected_blocks.py:11-101 there), int32 and int64 IDs,
duplicates, negative and out-of-range IDs, kb < qb and kb > qb, sinks, rows
wider than the candidate list, and a cfg5-sized grid (4 KV heads x 2048
query blocks, 96 candidates per row).  Every output row must also pass the
selected_blocks validator.
"""
import numpy as np
import pytest
import torch

import oracle.packing as op
from interfaces.packing import selected_ids_to_blocks, selected_mask_to_blocks
from interfaces.validator import validate_selected_blocks

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_reference_known_answers():
    sel = torch.zeros((2, 2, 4, 4), dtype=torch.bool)
    sel[..., 0, 0] = sel[..., 1, 0] = sel[..., 2, 0] = sel[..., 3, 0] = sel[..., 3, 1] = True
    packed = selected_mask_to_blocks(sel.to(DEV), k_selected=3, local_window=1).cpu()
    assert packed.shape == (1, 2, 2, 4, 3)
    assert packed[0, 0, 0].tolist() == [[0, -1, -1], [0, 1, -1], [0, 1, 2], [0, 2, 3]]
    validate_selected_blocks(packed)
    ids = torch.tensor([[[[5, 5], [5, 5], [5, 5], [2, 5], [2, 3], [3, 4]]]], dtype=torch.long)
    with_sink = selected_ids_to_blocks(ids.to(DEV), k_selected=4, local_window=1, key_blocks=6, sink_blocks=1).cpu()
    assert [with_sink[0, 0, 0, r, 0].item() for r in range(6)] == [0] * 6
    validate_selected_blocks(with_sink)
    packed = selected_ids_to_blocks(torch.full((1, 1, 4, 2), -1, device=DEV), 3, 1, 4, sink_blocks=1).cpu()
    assert packed[0, 0, 0, :2].tolist() == [[0, -1, -1], [0, 1, -1]]
    with pytest.raises(ValueError, match="cannot fit local window"):
        selected_mask_to_blocks(torch.ones((1, 1, 3, 3), dtype=torch.bool, device=DEV), k_selected=1)
    with pytest.raises(ValueError, match="sink block"):
        selected_ids_to_blocks(torch.zeros((1, 1, 4, 2), dtype=torch.long, device=DEV), 2, 1, 4, sink_blocks=1)


@pytest.mark.parametrize("seed,L,G,qb,kb,C,k,lw,sink,dtype", [
    (0, 2, 3, 9, 9, 5, 4, 1, 0, torch.int64),
    (1, 1, 4, 12, 7, 8, 6, 2, 1, torch.int32),
    (2, 2, 2, 6, 11, 3, 8, 0, 3, torch.int64),
    (3, 1, 1, 70, 70, 130, 20, 1, 2, torch.int32),      # more candidates than one wave, duplicates
    (4, 3, 2, 5, 5, 1, 2, 1, 0, torch.int32),
    (5, 1, 4, 300, 300, 64, 40, 3, 4, torch.int64),     # bitmap wider than 64 words
    (6, 1, 2, 40, 40, 2, 16, 1, 0, torch.int32),        # width C+lw+1 < k
])
def test_ids_match_oracle(seed, L, G, qb, kb, C, k, lw, sink, dtype):
    rng = np.random.default_rng(seed)
    ids = rng.integers(-3, max(qb, kb) + 3, size=(L, G, qb, C))
    if seed == 3:
        ids[..., 1::2] = ids[..., ::2][..., : ids[..., 1::2].shape[-1]]   # planted duplicates
    got = selected_ids_to_blocks(torch.from_numpy(ids).to(dtype).to(DEV), k, lw, kb, sink).cpu().numpy()
    exp = op.pack_ids(ids, k, lw, kb, sink)
    assert got.shape == exp.shape and np.array_equal(got, exp)
    if kb >= qb and lw == 1:
        validate_selected_blocks(torch.from_numpy(got))


@pytest.mark.parametrize("seed,L,G,qb,kb,k,lw,density", [
    (0, 2, 3, 9, 9, 4, 1, 0.3), (1, 1, 4, 12, 7, 6, 2, 0.5), (2, 2, 2, 6, 11, 8, 0, 0.4),
    (3, 1, 2, 200, 200, 24, 1, 0.2), (4, 1, 1, 33, 33, 33, 1, 1.0), (5, 1, 3, 130, 130, 9, 3, 0.02),
])
def test_mask_match_oracle(seed, L, G, qb, kb, k, lw, density):
    rng = np.random.default_rng(seed)
    mask = rng.random((L, G, qb, kb)) < density
    got = selected_mask_to_blocks(torch.from_numpy(mask).to(DEV), k, lw).cpu().numpy()
    exp = op.pack_mask(mask, k, lw)
    assert got.shape == exp.shape and np.array_equal(got, exp)


def test_cfg5_sized_grid_and_round_trip():
    rng = np.random.default_rng(11)
    qb, C, k = 2048, 96, 64
    ids = rng.integers(0, qb, size=(1, 4, qb, C))
    got = selected_ids_to_blocks(torch.from_numpy(ids).to(DEV), k, 1, None, 1).cpu()
    assert np.array_equal(got.numpy(), op.pack_ids(ids, k, 1, None, 1))
    validate_selected_blocks(got)
    # Round trip: a packed row, re-packed as IDs or as its mask, is unchanged.
    again = selected_ids_to_blocks(got[0].to(DEV), k, 1, None, 1).cpu()
    assert torch.equal(again[..., : got.shape[-1]], got)
    dense = torch.zeros((1, 4, qb, qb + 1), dtype=torch.bool)
    dense.scatter_(-1, got[0].long().masked_fill(got[0] < 0, qb), True)
    rem = selected_mask_to_blocks(dense[..., :qb].to(DEV), k, 1).cpu()
    assert got.shape[-1] == k and torch.equal(rem, got)
