"""Residual summaries on the GPU: the frontier kernel (spruce_residual_frontier)
bit-exact against the oracle, and sparse prefill with summary keys
(spruce_sparse_prefill_index_summaries) against the float32 oracle.

Bars: frontier node lists are integers and must match exactly; attention
outputs within max-abs 2e-2 / mean-abs 1e-3 of the oracle, whose summary
table is the float64 oracle table over the same K/V.  Full-size (cfg2
shape, T=32768) is checked through the size-independent partition and
maximality properties for every row, and on sampled query blocks against
the oracle.
"""
import numpy as np
import pytest
import torch

import oracle.attention as ora
import oracle.summaries as osum
from interfaces.residual_summaries import (
    build_residual_summary_nodes,
    build_residual_tree_layout,
    validate_residual_summary_nodes,
)
from kernels.direct_index import direct_index_sparse_prefill
from sparse.attention import sparse_prefill_attention_forward
from spruce_hip import workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
MAX_ABS, MEAN_ABS = 2e-2, 1e-3


class _Module(torch.nn.Module):
    layer_idx = 0


def _routes(num_blocks=5):
    selected = torch.full((1, 1, 1, num_blocks, 2), -1, dtype=torch.int32)
    for q in range(num_blocks):
        vals = torch.arange(max(0, q - 1), q + 1, dtype=torch.int32)
        selected[0, 0, 0, q, : len(vals)] = vals
    return selected


def test_reference_routes_table():
    for device in ("cpu", DEV):
        residual = build_residual_summary_nodes(_routes().to(device))
        assert residual.device.type == torch.device(device).type
        assert residual.shape == (1, 1, 1, 5, 2)
        assert residual[0, 0, 0].tolist() == [[-1, -1], [-1, -1], [0, -1], [5, -1], [2, 5]]
        validate_residual_summary_nodes(_routes().to(device), residual)


def test_all_exact_route_has_zero_width():
    Q = 4
    selected = torch.full((1, 1, 1, Q, Q), -1, dtype=torch.int32)
    for q in range(Q):
        selected[0, 0, 0, q, : q + 1] = torch.arange(q + 1, dtype=torch.int32)
    residual = build_residual_summary_nodes(selected.to(DEV))
    assert residual.shape == (1, 1, 1, Q, 0)


def test_non_causal_ids_raise():
    selected = _routes().to(DEV)
    selected[0, 0, 0, 2, 1] = 4
    with pytest.raises(ValueError, match="causal"):
        build_residual_summary_nodes(selected, validate_selected=False)


@pytest.mark.parametrize("qblocks", [1, 3, 5, 64, 129, 300, 1000])
def test_random_rows_match_oracle(qblocks):
    rng = np.random.default_rng(qblocks)
    B, L, G, K = 2, 2, 2, 12
    sel = np.full((B, L, G, qblocks, K), -1, np.int32)
    for idx in np.ndindex(B, L, G, qblocks):
        q = idx[3]
        n = rng.integers(0, K + 1)
        row = rng.integers(-3, q + 1, size=n)  # negatives ignored, duplicates, any order
        sel[idx][:n] = row
    # Non-contiguous strides: a transposed copy viewed back.
    selected = torch.from_numpy(sel).to(DEV).transpose(1, 2).contiguous().transpose(1, 2)
    out = build_residual_summary_nodes(selected, validate_selected=False).cpu().numpy()
    width = 0
    for idx in np.ndindex(B, L, G, qblocks):
        expected = osum.frontier_dyadic(sel[idx].tolist(), idx[3], qblocks)
        width = max(width, len(expected))
        got = out[idx]
        assert got[: len(expected)].tolist() == expected, idx
        assert (got[len(expected):] == -1).all(), idx
    assert out.shape[-1] == width


def _cfg2_selected(T=32768, Hkv=4, Hq=28):
    mask, _ = workloads.cfg2_mask(0, T=T, Hq=Hq, Hkv=Hkv)
    return workloads.mask_to_selected_blocks(mask[:, :: Hq // Hkv])[:, None]  # [1,1,Hkv,Qb,K]


def test_cfg2_frontier_partition_and_sampled_rows():
    selected = _cfg2_selected().to(DEV)
    residual = build_residual_summary_nodes(selected)
    print(f"cfg2 frontier width {residual.shape[-1]}", flush=True)
    validate_residual_summary_nodes(selected, residual)
    res, sel = residual.cpu().numpy(), selected.cpu().numpy()
    for g in range(4):
        for q in (0, 1, 2, 3, 4, 100, 257, 511):
            expected = osum.frontier_dyadic(sel[0, 0, g, q].tolist(), q, 512)
            row = res[0, 0, g, q]
            assert row[row >= 0].tolist() == expected


def _summary_case(seed, B, Hq, Hkv, T, D, dtype, extra):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, Hq, D, generator=gen).to(dtype).transpose(1, 2)
    k = torch.randn(B, T, Hkv, D, generator=gen).to(dtype).transpose(1, 2)
    v = torch.randn(B, T, Hkv, D, generator=gen).to(dtype).transpose(1, 2)
    Q = (T + 63) // 64
    rng = np.random.default_rng(seed)
    K = extra + 2
    sel = np.full((B, 1, Hkv, Q, K), -1, np.int32)
    for b, g, qb in np.ndindex(B, Hkv, Q):
        pick = rng.choice(qb + 1, size=min(qb + 1, extra), replace=False).tolist()
        row = sorted(set(pick) | {qb, max(0, qb - 1)})
        sel[b, 0, g, qb, : len(row)] = row
    return q, k, v, torch.from_numpy(sel)


def _oracle(q, k, v, selected, residual, P, qblocks_subset=None):
    qn, kn, vn = (x.float().numpy() for x in (q, k, v))
    Q = selected.shape[3]
    lay = osum.tree_layout(Q)
    rs, re = osum.token_ranges(lay["starts"], lay["ends"], kn.shape[2], 64, P)
    keys, vals, _, logc = osum.kv_summary(kn, vn, rs, re)
    B, H, _, D = kn.shape
    N = len(lay["starts"])
    return ora.sparse_attention_summaries(
        qn, kn, vn, selected[:, 0].numpy(), residual[:, 0].cpu().numpy(),
        keys.reshape(B, H, N, P, D), vals.reshape(B, H, N, P, D), logc.reshape(B, N, P),
        qblocks_subset=qblocks_subset)


@pytest.mark.parametrize("B,Hq,Hkv,T,D,dtype,P,extra", [
    (1, 8, 2, 300, 128, torch.bfloat16, 1, 2),
    (1, 8, 2, 1000, 128, torch.bfloat16, 4, 3),
    (2, 4, 4, 517, 64, torch.float16, 2, 1),
    (1, 28, 4, 777, 128, torch.bfloat16, 4, 4),
    (1, 6, 2, 450, 128, torch.float32, 2, 2),
])
def test_summary_attention_matches_oracle(B, Hq, Hkv, T, D, dtype, P, extra):
    q, k, v, selected = _summary_case(B * T + P, B, Hq, Hkv, T, D, dtype, extra)
    residual = build_residual_summary_nodes(selected.to(DEV))
    assert residual.shape[-1] > 0
    qd, kd, vd = (x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v))
    out, _ = sparse_prefill_attention_forward(
        _Module(), qd, kd, vd, None, selected_blocks=selected.to(DEV), block_size=64,
        residual_summaries=True, residual_summary_nodes=residual, summary_prototypes=P)
    torch.cuda.synchronize()
    expected = _oracle(q, k, v, selected, residual, P)
    a = out.float().cpu().numpy()
    assert np.isfinite(a).all()
    d = np.abs(a.astype(np.float64) - expected)
    print(f"summaries B={B} Hq={Hq} T={T} D={D} {dtype} P={P}: max_abs={d.max():.3e} "
          f"mean_abs={d.mean():.3e}", flush=True)
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS
    # The summaries change the result (the route omits blocks).
    plain = direct_index_sparse_prefill(qd, kd, vd, selected[:, 0].to(DEV), scale=D ** -0.5)
    assert (plain.float() - out.float()).abs().max().item() > 1e-2


def test_identical_keys_make_summaries_exact():
    # The reference's multiplicity check at block size 64: identical keys, so
    # exact blocks + log(count)-weighted summaries == dense causal attention.
    gen = torch.Generator().manual_seed(4)
    T, Hq, Hkv, D = 640, 4, 1, 64
    q = torch.randn(1, Hq, T, D, generator=gen).to(torch.bfloat16)
    k = torch.ones(1, Hkv, T, D, dtype=torch.bfloat16)
    v = torch.randn(1, Hkv, T, D, generator=gen).to(torch.bfloat16)
    Q = T // 64
    sel = torch.full((1, 1, 1, Q, 2), -1, dtype=torch.int32)
    for qb in range(Q):
        row = torch.arange(max(0, qb - 1), qb + 1, dtype=torch.int32)
        sel[0, 0, 0, qb, : len(row)] = row
    for P in (1, 2, 4):
        residual = build_residual_summary_nodes(sel.to(DEV))
        out, _ = sparse_prefill_attention_forward(
            _Module(), q.to(DEV), k.to(DEV), v.to(DEV), None, selected_blocks=sel.to(DEV),
            block_size=64, residual_summaries=True, residual_summary_nodes=residual,
            summary_prototypes=P)
        dense = ora.dense_causal_attention(q.float().numpy(), k.float().numpy(), v.float().numpy())
        d = np.abs(out.float().cpu().numpy() - dense)
        print(f"identical keys P={P}: max_abs={d.max():.3e} mean_abs={d.mean():.3e}", flush=True)
        assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS


def test_empty_frontier_is_bit_identical_to_plain():
    gen = torch.Generator().manual_seed(9)
    T, Hq, Hkv, D = 320, 8, 2, 128
    q, k, v = (torch.randn(1, H, T, D, generator=gen).to(torch.bfloat16).to(DEV) for H in (Hq, Hkv, Hkv))
    Q = T // 64
    sel = torch.full((1, 1, Hkv, Q, Q), -1, dtype=torch.int32)
    for qb in range(Q):
        sel[0, 0, :, qb, : qb + 1] = torch.arange(qb + 1, dtype=torch.int32)
    residual = build_residual_summary_nodes(sel.to(DEV))
    assert residual.shape[-1] == 0
    out, _ = sparse_prefill_attention_forward(
        _Module(), q, k, v, None, selected_blocks=sel.to(DEV), block_size=64,
        residual_summaries=True, residual_summary_nodes=residual, summary_prototypes=4)
    plain, _ = sparse_prefill_attention_forward(
        _Module(), q, k, v, None, selected_blocks=sel.to(DEV), block_size=64)
    assert torch.equal(out, plain)


def test_entry_point_errors():
    q, k, v, selected = _summary_case(1, 1, 4, 2, 320, 64, torch.bfloat16, 0)
    qd, kd, vd, sd = q.to(DEV), k.to(DEV), v.to(DEV), selected.to(DEV)
    with pytest.raises(ValueError, match="requires residual_summary_nodes"):
        sparse_prefill_attention_forward(_Module(), qd, kd, vd, None, selected_blocks=sd, block_size=64,
                                         residual_summaries=True)
    residual = build_residual_summary_nodes(sd)
    with pytest.raises(ValueError, match="summary_checkpoint"):
        sparse_prefill_attention_forward(_Module(), qd, kd, vd, None, selected_blocks=sd, block_size=64,
                                         residual_summaries=True, residual_summary_nodes=residual,
                                         summary_mode="learned")
    bad = residual.clone()
    bad[0, 0, 0, 1, 0] = 0  # row q=1 selects block 0 itself: overlap
    with pytest.raises(AssertionError, match="partition|Duplicate|not maximal"):
        sparse_prefill_attention_forward(_Module(), qd, kd, vd, None, selected_blocks=sd, block_size=64,
                                         residual_summaries=True, residual_summary_nodes=bad)


def test_cfg2_full_size_sampled_rows():
    T, Hq, Hkv, D = 32768, 28, 4, 128
    q, k, v = workloads.qkv(0, T, Hq, Hkv, D, torch.bfloat16, use_rope=True, layout="bthd")
    selected = _cfg2_selected(T, Hkv, Hq)
    sd = selected.to(DEV)
    residual = build_residual_summary_nodes(sd)
    qd, kd, vd = (x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v))
    out, _ = sparse_prefill_attention_forward(
        _Module(), qd, kd, vd, None, selected_blocks=sd, block_size=64,
        residual_summaries=True, residual_summary_nodes=residual, summary_prototypes=4,
        validate_residual_summary_nodes_input=False)
    torch.cuda.synchronize()
    blocks = [0, 3, 97, 300, 511]
    expected = _oracle(q, k, v, selected, residual, 4, qblocks_subset=blocks)
    a = out.float().cpu().numpy()
    assert np.isfinite(a).all()
    for qb in blocks:
        sl = slice(qb * 64, (qb + 1) * 64)
        d = np.abs(a[:, sl].astype(np.float64) - expected[:, sl])
        print(f"cfg2 summaries qb={qb}: max_abs={d.max():.3e} mean_abs={d.mean():.3e}", flush=True)
        assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS
