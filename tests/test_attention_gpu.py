"""Parity of the gfx950 sparse-prefill kernels (through the C ABI) with the
CPU oracle on identical seeded inputs.

Bar (north star): max-abs error <= 2e-2 and mean-abs error <= 1e-3 against
the float32 oracle; the reference's own Triton parity cases additionally use
its torch.testing tolerance atol = rtol = 2e-2
(tests/test_triton_sparse_prefill.py:94,125 in the reference).  Full size:
cfg2 and cfg5 on every row (cfg5 in chunks of 256 query blocks), and
size-independent properties: the three list layouts and the
dispatch order give bit-identical outputs for identical block sets.
"""
import numpy as np
import pytest
import torch

import oracle.attention as ora
from kernels.block_mask import block_sparse_prefill
from kernels.direct_index import (
    KERNEL_VARIANTS,
    csr_row_order,
    direct_index_sparse_csr,
    direct_index_sparse_prefill,
    kernel_runtime_metadata,
)
from kernels.sparse_prefill import triton_sparse_prefill_attention_forward
from sparse.attention import sparse_prefill_attention_forward
from spruce_hip import workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
MAX_ABS, MEAN_ABS = 2e-2, 1e-3


class _Module(torch.nn.Module):
    layer_idx = 0


def _err(actual, expected):
    a = actual.detach().float().cpu().numpy().astype(np.float64)
    d = np.abs(a - np.asarray(expected, dtype=np.float64))
    return float(d.max()), float(d.mean())


def _assert_parity(actual, expected, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what=""):
    mx, mn = _err(actual, expected)
    print(f"{what}: max_abs={mx:.3e} mean_abs={mn:.3e}", flush=True)
    assert np.isfinite(actual.float().cpu().numpy()).all(), what
    assert mx <= max_abs and mn <= mean_abs, (what, mx, mn)


def _bthd(B, T, H, D, dtype, gen):
    """Qwen projection layout: contiguous [B,T,H,D] viewed as [B,H,T,D]."""
    return torch.randn(B, T, H, D, generator=gen).to(dtype).transpose(1, 2)


@pytest.mark.parametrize("variant", KERNEL_VARIANTS)
def test_reference_parity_case_one_block(variant):
    # Reference tests/test_triton_sparse_prefill.py:74-95 (fp16, strided views).
    torch.manual_seed(0)
    q = torch.randn(1, 64, 2, 64, dtype=torch.float16).transpose(1, 2)
    k = torch.randn(1, 64, 1, 64, dtype=torch.float16).transpose(1, 2)
    v = torch.randn(1, 64, 1, 64, dtype=torch.float16).transpose(1, 2)
    assert not q.is_contiguous()
    selected = torch.zeros((1, 1, 1, 1, 1), dtype=torch.int32)
    expected = ora.sparse_attention_index(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                          selected[:, 0].numpy())
    qd, kd, vd = (x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v))
    actual, _ = triton_sparse_prefill_attention_forward(
        _Module(), qd, kd, vd, None, selected_blocks=selected.to(DEV), block_size=64,
        kernel_variant=variant)
    assert actual.shape == (1, 64, 2, 64) and actual.is_contiguous()
    torch.testing.assert_close(actual.float().cpu(), torch.from_numpy(expected), atol=2e-2, rtol=2e-2)
    assert kernel_runtime_metadata(variant)["best_config"] is not None


@pytest.mark.parametrize("variant", KERNEL_VARIANTS)
def test_reference_parity_case_across_blocks(variant):
    # Reference tests/test_triton_sparse_prefill.py:103-125.
    torch.manual_seed(4)
    q = torch.randn(1, 128, 4, 64, dtype=torch.float16).transpose(1, 2)
    k = torch.randn(1, 128, 2, 64, dtype=torch.float16).transpose(1, 2)
    v = torch.randn(1, 128, 2, 64, dtype=torch.float16).transpose(1, 2)
    selected = torch.tensor([[[[[0, -1], [0, 1]], [[0, -1], [0, 1]]]]], dtype=torch.int32)
    expected = ora.sparse_attention_index(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                          selected[:, 0].numpy())
    qd, kd, vd = (x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v))
    actual, _ = triton_sparse_prefill_attention_forward(
        _Module(), qd, kd, vd, None, selected_blocks=selected.to(DEV), block_size=64,
        kernel_variant=variant)
    torch.testing.assert_close(actual.float().cpu(), torch.from_numpy(expected), atol=2e-2, rtol=2e-2)


def test_cfg1_block_mask_fp32_inputs():
    # Benchmark configuration cfg1: T=4096, 8q/2kv, d=128, fp32 N(0,1), top-16 + sink + diagonal.
    q, k, v = workloads.qkv(0, 4096, 8, 2, 128, torch.float32, use_rope=False)
    mask = workloads.cfg1_mask(0)
    expected = ora.sparse_attention_mask(q.numpy(), k.numpy(), v.numpy(), mask.numpy())
    actual = block_sparse_prefill(q.to(DEV), k.to(DEV), v.to(DEV), mask.to(DEV), scale=128 ** -0.5)
    _assert_parity(actual.transpose(1, 2), expected, what="cfg1 mask fp32")


def _messy_index_rows(rng, B, Hkv, qblocks, K):
    idx = np.full((B, Hkv, qblocks, K), -1, np.int32)
    for b in range(B):
        for g in range(Hkv):
            for qb in range(qblocks):
                n = rng.integers(0, K + 1)
                row = list(rng.integers(-1, qblocks + 2, size=n))   # -1, dups, future ids
                if rng.random() < 0.8:
                    row.append(qb)
                row = row[:K]
                rng.shuffle(row)
                idx[b, g, qb, : len(row)] = row
    return idx


@pytest.mark.parametrize("B,Hq,Hkv,T,D,dtype", [
    (2, 14, 2, 1000, 128, torch.bfloat16),   # G=7, ragged last block
    (1, 8, 2, 777, 64, torch.float16),       # G=4, D=64
    (1, 3, 3, 300, 128, torch.float32),      # G=1, fp32 inputs
    (1, 12, 2, 640, 128, torch.bfloat16),    # G=6 (Qwen2.5-1.5B grouping)
])
def test_direct_index_messy_rows(B, Hq, Hkv, T, D, dtype):
    rng = np.random.default_rng(B * 1000 + Hq * 10 + D)
    gen = torch.Generator().manual_seed(int(T))
    q = _bthd(B, T, Hq, D, dtype, gen)
    k = _bthd(B, T, Hkv, D, dtype, gen)
    v = _bthd(B, T, Hkv, D, dtype, gen)
    qblocks = (T + 63) // 64
    idx = _messy_index_rows(rng, B, Hkv, qblocks, 6)
    expected = ora.sparse_attention_index(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                          idx, empty="zero")
    dev = [x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v)]
    actual = direct_index_sparse_prefill(*dev, torch.from_numpy(idx).to(DEV), scale=D ** -0.5)
    _assert_parity(actual, expected, what=f"index B{B} Hq{Hq} Hkv{Hkv} T{T} D{D} {dtype}")


@pytest.mark.parametrize("variant", ["single_head_qtile", "single_head_prescale", "tiled_gqa"])
def test_variants_agree_with_oracle(variant):
    gen = torch.Generator().manual_seed(17)
    q = _bthd(1, 512, 28, 128, torch.bfloat16, gen)
    k = _bthd(1, 512, 4, 128, torch.bfloat16, gen)
    v = _bthd(1, 512, 4, 128, torch.bfloat16, gen)
    idx = torch.tensor([[[[0, q_, -1] if q_ else [0, -1, -1] for q_ in range(8)]] * 4], dtype=torch.int32)
    expected = ora.sparse_attention_index(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                          idx.numpy())
    dev = [x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v)]
    actual = direct_index_sparse_prefill(*dev, idx.to(DEV), scale=128 ** -0.5, kernel_variant=variant)
    _assert_parity(actual, expected, what=variant)


def test_csr_rows_with_row_order_and_empty_rows():
    rng = np.random.default_rng(23)
    B, Hq, Hkv, T, D = 1, 8, 2, 700, 64
    gen = torch.Generator().manual_seed(3)
    q = _bthd(B, T, Hq, D, torch.float16, gen)
    k = _bthd(B, T, Hkv, D, torch.float16, gen)
    v = _bthd(B, T, Hkv, D, torch.float16, gen)
    qblocks = (T + 63) // 64
    rows = []
    for _ in range(B * Hkv * qblocks):
        rows.append(rng.integers(-1, qblocks, size=rng.integers(0, 9)).astype(np.int32))
    indptr = np.concatenate([[0], np.cumsum([r.size for r in rows])]).astype(np.int32)
    indices = np.concatenate(rows).astype(np.int32)
    expected = ora.sparse_attention_csr(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                        indptr, indices, empty="zero")
    dev = [x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v)]
    ip, ix = torch.from_numpy(indptr).to(DEV), torch.from_numpy(indices).to(DEV)
    plain = direct_index_sparse_csr(*dev, ip, ix, scale=D ** -0.5)
    ordered = direct_index_sparse_csr(*dev, ip, ix, scale=D ** -0.5, row_order=csr_row_order(ip, Hkv))
    _assert_parity(plain, expected, what="csr")
    assert torch.equal(plain, ordered)


@pytest.mark.parametrize("T", [1, 100])
def test_csr_with_no_entries_writes_zeros(T):
    # Every row empty: nnz = 0 and an empty (null) indices tensor.
    gen = torch.Generator().manual_seed(T)
    dev = [_bthd(2, T, H, 64, torch.bfloat16, gen).transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
           for H in (4, 2, 2)]
    rows = 2 * 2 * ((T + 63) // 64)
    indptr = torch.zeros(rows + 1, dtype=torch.int32, device=DEV)
    indices = torch.zeros(0, dtype=torch.int32, device=DEV)
    out = direct_index_sparse_csr(*dev, indptr, indices, scale=0.125)
    torch.cuda.synchronize()
    assert out.shape == (2, T, 4, 64) and not out.float().abs().any()


def test_mask_per_query_head_and_per_kv_head():
    rng = np.random.default_rng(31)
    B, Hq, Hkv, T, D = 1, 8, 2, 512, 128
    gen = torch.Generator().manual_seed(5)
    q = torch.randn(B, Hq, T, D, generator=gen).to(torch.bfloat16)
    k = torch.randn(B, Hkv, T, D, generator=gen).to(torch.bfloat16)
    v = torch.randn(B, Hkv, T, D, generator=gen).to(torch.bfloat16)
    qblocks = T // 64
    per_q = rng.random((B, Hq, qblocks, qblocks)) < 0.4   # heads of a group differ
    per_q[0, 1, 3] = False                                 # one empty (head, row): zeros
    per_kv = rng.random((B, Hkv, qblocks, qblocks)) < 0.4
    for m in (per_q, per_kv):
        expected = ora.sparse_attention_mask(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                             m, empty="zero")
        actual = block_sparse_prefill(q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(m).to(DEV),
                                      scale=D ** -0.5)
        _assert_parity(actual.transpose(1, 2), expected, what=f"mask heads={m.shape[1]}")


def test_reference_shaped_mask_call_with_expanded_kv():
    # The reference kernel requires q.shape == k.shape (GQA pre-expanded).
    gen = torch.Generator().manual_seed(8)
    q = torch.randn(1, 4, 256, 64, generator=gen).to(torch.float16)
    k = torch.randn(1, 4, 256, 64, generator=gen).to(torch.float16)
    v = torch.randn(1, 4, 256, 64, generator=gen).to(torch.float16)
    mask = torch.tril(torch.ones(4, 4, dtype=torch.bool))[None, None].expand(1, 4, 4, 4).contiguous()
    expected = ora.dense_causal_attention(q.float().numpy(), k.float().numpy(), v.float().numpy())
    actual = block_sparse_prefill(q.to(DEV), k.to(DEV), v.to(DEV), mask.to(DEV), scale=64 ** -0.5)
    _assert_parity(actual.transpose(1, 2), expected, what="all-causal mask == dense")


def test_sparse_attention_entry_point_drop_in():
    gen = torch.Generator().manual_seed(2)
    q = _bthd(1, 256, 4, 128, torch.bfloat16, gen)
    k = _bthd(1, 256, 2, 128, torch.bfloat16, gen)
    v = _bthd(1, 256, 2, 128, torch.bfloat16, gen)
    rows = [[0, -1], [0, 1], [1, 2], [2, 3]]
    sel = torch.tensor([[[rows, rows]]], dtype=torch.int32)   # [B=1, L=1, Hkv=2, Qb=4, K=2]
    expected = ora.sparse_attention_index(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                          sel[:, 0].numpy())
    dev = [x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v)]
    actual, w = sparse_prefill_attention_forward(_Module(), *dev, None, selected_blocks=sel.to(DEV),
                                                 block_size=64)
    assert w is None
    _assert_parity(actual, expected, what="sparse/attention.py")
    bad = sel.clone()
    bad[0, 0, 1, 2] = -1
    with pytest.raises(ValueError, match="row empty"):
        sparse_prefill_attention_forward(_Module(), *dev, None, selected_blocks=bad.to(DEV),
                                         block_size=64, validate_selected_blocks_input=False)
    # Under inference_mode (how the reference's scripts run the model) the
    # route is an inference tensor without a version counter.
    with torch.inference_mode():
        sel_i = sel.to(DEV)
        again, _ = sparse_prefill_attention_forward(_Module(), *dev, None, selected_blocks=sel_i,
                                                    block_size=64)
        assert torch.equal(again, actual)
        sel_i[0, 0, 1, 2] = -1
        with pytest.raises(ValueError, match="row empty"):
            sparse_prefill_attention_forward(_Module(), *dev, None, selected_blocks=sel_i,
                                             block_size=64, validate_selected_blocks_input=False)


def test_full_size_cfg2_every_row_and_layout_identity():
    # Benchmark configuration cfg2 at full size: T=32768, 28q/4kv, bf16 + RoPE, ~10% density.
    print("cfg2: generating inputs", flush=True)
    q, k, v = workloads.qkv(0, 32768, 28, 4, 128, torch.bfloat16, use_rope=True, layout="bthd")
    mask, density = workloads.cfg2_mask(0)
    assert 0.09 < density < 0.12
    dev = [x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v)]
    mask_d = mask.to(DEV)
    by_mask = block_sparse_prefill(*dev, mask_d, scale=128 ** -0.5)
    sel = workloads.mask_to_selected_blocks(mask[:, ::7]).to(DEV)
    by_index = direct_index_sparse_prefill(*dev, sel, scale=128 ** -0.5)
    torch.cuda.synchronize()
    # Same blocks in the same ascending order -> bit-identical results.
    assert torch.equal(by_mask.transpose(1, 2).contiguous(), by_index)
    print("cfg2: oracle on all 512 query blocks", flush=True)
    expected = ora.sparse_attention_mask(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                         mask[:, ::7].numpy())
    _assert_parity(by_index, expected, what="cfg2 every row")


def test_full_size_cfg5_csr_every_row():
    # Benchmark configuration cfg5 at full size: T=131072 CSR, log-normal density (median 2%).
    # Every query block of every KV head against the oracle, in chunks of 256
    # query blocks (a progress line after each).
    print("cfg5: generating inputs", flush=True)
    q, k, v = workloads.qkv(0, 131072, 28, 4, 128, torch.bfloat16, use_rope=True,
                            layout="bthd", device=DEV)
    indptr, indices = workloads.cfg5_csr(0)
    ip, ix = indptr.to(DEV), indices.to(DEV)
    out = direct_index_sparse_csr(q, k, v, ip, ix, scale=128 ** -0.5, row_order=csr_row_order(ip, 4))
    out_plain = direct_index_sparse_csr(q, k, v, ip, ix, scale=128 ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(out, out_plain)
    out = out.cpu()
    qf = q.float().cpu().numpy()
    kf, vf = k.float().cpu().numpy(), v.float().cpu().numpy()
    ipn, ixn = indptr.numpy(), indices.numpy()
    worst = 0.0
    for c0 in range(0, 2048, 256):
        sample = list(range(c0, c0 + 256))
        rows = np.arange(c0 * 64, (c0 + 256) * 64)
        qs = np.zeros_like(qf)
        qs[:, :, rows] = qf[:, :, rows]
        expected = ora.sparse_attention_csr(qs, kf, vf, ipn, ixn, qblocks_subset=sample)
        d = np.abs(out[:, rows].double().numpy() - expected[:, rows])
        worst = max(worst, float(d.max()))
        _assert_parity(out[:, rows], expected[:, rows], what=f"cfg5 query blocks {c0}..{c0 + 255}")
    print(f"cfg5: every row within the bar (max_abs {worst:.3e})", flush=True)


@pytest.mark.parametrize("variant", ["single_head", "single_head_qtile"])
@pytest.mark.parametrize("Hq,Hkv", [
    (28, 4),   # G=7, Qwen2-7B: two 8-wave parts of 7 tiles (half-major)
    (20, 4),   # G=5
    (24, 4),   # G=6
    (32, 4),   # G=8: two full 8-wave parts (half-major)
    (12, 4),   # G=3: one part, 6 tiles of 3 heads
    (20, 2),   # G=10: 8-wave parts, head-major order
    (24, 2),   # G=12: three 8-wave parts, the middle one wraps to head 0
    (32, 2),   # G=16: four 8-wave parts
])
def test_mask_per_query_head_differs_within_group(Hq, Hkv, variant):
    # Per-query-head masks whose heads differ inside each KV group: every
    # part of a row must walk the mask rows of exactly the heads its tiles
    # hold (reference kernels/seerattention_triton.py:41-68 reads
    # mask[z, h, row, col] per head).
    G = Hq // Hkv
    rng = np.random.default_rng(Hq * 100 + Hkv)
    B, T, D = 1, 700, 128
    gen = torch.Generator().manual_seed(Hq + Hkv)
    q = _bthd(B, T, Hq, D, torch.bfloat16, gen)
    k = _bthd(B, T, Hkv, D, torch.bfloat16, gen)
    v = _bthd(B, T, Hkv, D, torch.bfloat16, gen)
    qblocks = (T + 63) // 64
    mask = rng.random((B, Hq, qblocks, qblocks)) < 0.35
    # Blocks that only the last head of each group selects, so a part that
    # misses that head's row skips them.
    for g in range(Hkv):
        mask[:, g * G:(g + 1) * G - 1, :, 2] = False
        mask[:, (g + 1) * G - 1, 2:, 2] = True
    mask[0, 1, 4] = False   # one empty (head, row): zeros
    expected = ora.sparse_attention_mask(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                         mask, empty="zero")
    dev = [x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v)]
    actual = block_sparse_prefill(*dev, torch.from_numpy(mask).to(DEV), scale=D ** -0.5,
                                  kernel_variant=variant)
    _assert_parity(actual.transpose(1, 2), expected, what=f"per-head mask G={G} {variant}")


def _ascending_route(rng, B, L, Hkv, qblocks, K):
    """[B, L, Hkv, Qb, K] int32 rows: sink 0 and the diagonal always listed,
    the rest a random causal subset, ascending, -1 padded."""
    route = np.full((B, L, Hkv, qblocks, K), -1, np.int32)
    for idx in np.ndindex(B, L, Hkv, qblocks):
        qb = idx[-1]
        extra = rng.permutation(np.arange(1, qb))[: rng.integers(0, K - 1)] if qb > 1 else []
        row = sorted({0, qb, *map(int, extra)})[:K]
        route[idx][: len(row)] = row
    return route


def test_route_adapters_on_device_feed_mask_and_index_kernels():
    # kernels/sparse_prefill.py:16-52 in the reference: the route -> block
    # mask and route -> per-query-head index adapters, run on device tensors
    # and fed to the HIP kernels.
    rng = np.random.default_rng(7)
    from kernels.sparse_prefill import selected_blocks_to_block_mask, selected_blocks_to_head_indices
    B, L, Hq, Hkv, T, D = 1, 2, 28, 4, 1000, 128
    G = Hq // Hkv
    qblocks = (T + 63) // 64
    route = _ascending_route(rng, B, L, Hkv, qblocks, 6)
    route_d = torch.from_numpy(route).to(DEV)
    gen = torch.Generator().manual_seed(11)
    q = _bthd(B, T, Hq, D, torch.bfloat16, gen)
    k = _bthd(B, T, Hkv, D, torch.bfloat16, gen)
    v = _bthd(B, T, Hkv, D, torch.bfloat16, gen)
    dev = [x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v)]

    mask_d = selected_blocks_to_block_mask(route_d, layer_idx=1, num_query_heads=Hq)
    heads_d = selected_blocks_to_head_indices(route_d, layer_idx=1, num_query_heads=Hq)
    assert mask_d.is_cuda and heads_d.is_cuda
    # The device adapters agree with the same adapters on the host.
    assert torch.equal(mask_d.cpu(), selected_blocks_to_block_mask(
        torch.from_numpy(route), layer_idx=1, num_query_heads=Hq))
    assert torch.equal(heads_d.cpu(), selected_blocks_to_head_indices(
        torch.from_numpy(route), layer_idx=1, num_query_heads=Hq))
    assert mask_d.shape == (B, Hq, qblocks, qblocks) and heads_d.shape == (B, Hq, qblocks, 6)

    by_mask = block_sparse_prefill(*dev, mask_d, scale=D ** -0.5).transpose(1, 2).contiguous()
    by_index = direct_index_sparse_prefill(*dev, route_d[:, 1].contiguous(), scale=D ** -0.5)
    # Per-query-head rows run against K/V expanded to the query heads (the
    # reference's mask kernel takes expanded K/V the same way).
    k_exp = dev[1].repeat_interleave(G, dim=1)
    v_exp = dev[2].repeat_interleave(G, dim=1)
    by_heads = direct_index_sparse_prefill(dev[0], k_exp, v_exp, heads_d, scale=D ** -0.5)
    torch.cuda.synchronize()
    expected = ora.sparse_attention_index(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                          route[:, 1])
    _assert_parity(by_mask, expected, what="route -> mask")
    _assert_parity(by_index, expected, what="route -> index (KV heads)")
    _assert_parity(by_heads, expected, what="route -> per-query-head index")
    # Identical ascending block sets give identical arithmetic per tile.
    assert torch.equal(by_mask, by_index)
    assert torch.equal(by_heads, by_index)
