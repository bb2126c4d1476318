"""Host-side teacher utilities against the oracle: pool_attention, rollup and
check_causal (teacher/pool.py:3-39, teacher/validate.py:3-15 in the reference).

These run on any torch device; here on the CPU against oracle/teacher.py,
including the reference's own leak case (a 1e-3 cell above the diagonal).
"""
import numpy as np
import torch

import oracle.teacher as ot
from teacher.pool import pool_attention, rollup
from teacher.validate import check_causal


def test_pool_attention_matches_oracle_with_ragged_tails():
    a = torch.rand(2, 3, 100, 90, generator=torch.Generator().manual_seed(0), dtype=torch.float64)
    np.testing.assert_allclose(pool_attention(a, 8).numpy(), ot.pool_attention(a.numpy(), 8), atol=1e-12)


def test_rollup_levels_and_totals():
    p = torch.rand(1, 2, 12, 12, dtype=torch.float64)
    lv = rollup(p)
    ref = ot.rollup(p.numpy())
    assert [x.shape[-1] for x in lv] == [x.shape[-1] for x in ref] == [12, 6, 3]
    for a, b in zip(lv, ref):
        np.testing.assert_allclose(a.numpy(), b, atol=1e-12)
    assert len(rollup(torch.rand(1, 1, 5, 8))) == 1


def test_check_causal_first_leak_in_row_major_order():
    pooled = torch.zeros(1, 1, 3, 3)
    pooled[0, 0, 1, 2] = 1e-3
    assert check_causal(pooled) == (False, (1, 2)) == ot.check_causal(pooled.numpy())
    pooled[0, 0, 0, 2] = -5e-6
    assert check_causal(pooled) == (False, (0, 2))
    assert check_causal(torch.tril(torch.rand(2, 3, 6, 6))) == (True, None)
