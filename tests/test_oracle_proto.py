"""Pins the prototype-feature oracle (oracle/proto.c via oracle.selector).

Known answers are the reference's own tests of _proto_pool_seq and
_group_avg_tokens (tests/test_proto_pool.py:7-67 and tests/test_group_avg.py:7-15
in the reference): block mean as prototype 0, a planted needle kept among
the outliers in float32, float16 and bfloat16 (the fp16-overflow regression),
a ragged 3-row block padded with its mean, and per-group head means.
Beyond them: the model-dtype rounding equals torch's casts, and on random
blocks the oracle agrees with an independent float64 computation (means to
rounding, outlier rows equal to a float64 argsort wherever the distance gaps
are unambiguous).
"""
import numpy as np
import pytest
import torch

import oracle.selector as osel

_NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


def _pool(x, block, P, G=None):
    """Reference-shaped helper: torch [b,H,L,d] in a model dtype -> float32 numpy protos."""
    name = _NAMES[x.dtype]
    a = x.float().numpy()
    if G is not None:
        a = osel.group_avg(a, G, name)
    return osel.proto_pool(a, block, P, name)


def test_round_matches_torch_casts():
    x = (np.random.default_rng(0).standard_normal(50000) * 300).astype(np.float32)
    x[:4] = [1e-8, 6.1e-5, 65519.0, 70000.0]
    for dt in (torch.bfloat16, torch.float16):
        assert np.array_equal(osel.round_to(x, _NAMES[dt]), torch.from_numpy(x).to(dt).float().numpy())


def test_shape_and_mean():
    b, H, L, d, block, P = 1, 2, 128, 4, 64, 8
    x = torch.randn(b, H, L, d, generator=torch.Generator().manual_seed(0))
    out = _pool(x, block, P)
    assert out.shape == (b, H, 2, P, d)
    np.testing.assert_allclose(out[:, :, 0, 0, :], x[:, :, :block].mean(dim=2).numpy(), atol=1e-5)


def test_outlier_is_kept():
    x = torch.randn(1, 1, 64, 4, generator=torch.Generator().manual_seed(1)) * 0.01
    x[0, 0, 37, :] = 50.0
    protos = _pool(x, 64, 8)[0, 0, 0]
    assert ((protos - x[0, 0, 37].numpy()) ** 2).sum(-1).min() < 1e-6
    assert np.array_equal(protos[1], x[0, 0, 37].numpy())     # farthest first


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_needle_survives_reduced_precision(dtype):
    torch.manual_seed(0)
    x = (torch.randn(1, 1, 64, 128) * 0.01).to(dtype)
    x[0, 0, 37, :] = 40.0
    protos = _pool(x, 64, 8)[0, 0, 0]
    assert ((protos - x[0, 0, 37].float().numpy()) ** 2).sum(-1).min() < 1.0


def test_short_block_pads_with_mean():
    x = torch.randn(1, 1, 67, 4, generator=torch.Generator().manual_seed(2))
    last = _pool(x, 64, 8)[0, 0, 1]
    np.testing.assert_allclose(last[0], x[0, 0, 64:].mean(dim=0).numpy(), atol=1e-5)
    assert not (last == 0).all(axis=-1).any()
    assert all(np.array_equal(last[j], last[0]) for j in range(4, 8))   # 3 real outliers, 4 mean slots
    assert sorted(tuple(r) for r in last[1:4]) == sorted(tuple(r) for r in x[0, 0, 64:].numpy())


def test_group_average():
    x = torch.randn(1, 12, 10, 4, generator=torch.Generator().manual_seed(3))
    out = osel.group_avg(x.numpy(), 2, "float32")
    assert out.shape == (1, 2, 10, 4)
    np.testing.assert_allclose(out[:, 0], x[:, 0:6].mean(dim=1).numpy(), atol=1e-6)
    np.testing.assert_allclose(out[:, 1], x[:, 6:12].mean(dim=1).numpy(), atol=1e-6)
    xb = x.to(torch.bfloat16)
    ob = osel.group_avg(xb.float().numpy(), 2, "bfloat16")
    ref = xb.float().view(1, 2, 6, 10, 4).mean(dim=2).to(torch.bfloat16).float().numpy()
    assert np.abs(ob - ref).max() <= np.abs(ref).max() * 2 ** -7     # within one bf16 ulp


@pytest.mark.parametrize("dtype,L,d,block,P", [
    (torch.float32, 300, 16, 64, 8), (torch.bfloat16, 200, 32, 64, 8), (torch.float16, 90, 8, 16, 5),
])
def test_agrees_with_float64_closed_form(dtype, L, d, block, P):
    g = torch.Generator().manual_seed(L)
    x = torch.randn(1, 3, L, d, generator=g).to(dtype)
    out = _pool(x, block, P)
    a = x.double().numpy()
    nb = (L + block - 1) // block
    for h in range(3):
        for i in range(nb):
            rows = a[0, h, i * block:(i + 1) * block]
            m = rows.mean(axis=0)
            np.testing.assert_allclose(out[0, h, i, 0], m, atol=2e-2 if dtype != torch.float32 else 1e-5)
            dist = ((rows - m) ** 2).sum(-1)
            order = np.argsort(-dist, kind="stable")
            k = min(P - 1, rows.shape[0])
            srt = dist[order]
            for j in range(k):
                gap_ok = (j == 0 or srt[j - 1] - srt[j] > 1e-2 * srt[j]) and \
                         (j + 1 >= len(srt) or srt[j] - srt[j + 1] > 1e-2 * srt[j])
                if gap_ok:
                    assert np.array_equal(out[0, h, i, 1 + j], rows[order[j]].astype(np.float32)), (h, i, j)
