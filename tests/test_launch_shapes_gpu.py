"""Launch-shape invariance of the block-sparse entries.

A launch with fewer workgroups than the GPU has CUs splits each (batch, KV
head, query block) row into smaller parts (4 or 2 waves, one query tile per
wave); a larger batch of the same rows runs the 8-wave forms (with the K/V
producer wave for 16-bit inputs and 7 tiles per part).  Every shape computes
each tile with the same arithmetic in the same block order, so batch element
0 must come out bit-identical whether it runs alone (split) or as the first
of a batch (unsplit).  This keeps the 8-wave forms of every entry covered by
the small parity cases, and the small launch checked against the oracle.
"""
import numpy as np
import pytest
import torch

import oracle.attention as ora
from interfaces.residual_summaries import build_residual_summary_nodes, build_residual_tree_layout
from kernels.block_mask import block_sparse_prefill
from kernels.direct_index import (
    direct_index_sparse_csr,
    direct_index_sparse_prefill,
    direct_index_sparse_summaries,
)
from sparse.attention import sparse_prefill_attention_forward
from sparse.summaries import build_kv_summary_table

pytestmark = pytest.mark.gpu
DEV = "cuda"
T, D = 1024, 128
QB = T // 64

# (Hq, Hkv, batch that fills 256 CUs without splitting, dtype).  Alone, one
# batch element gives Hkv * 16 rows: 32 rows of 8 tiles (G=4) become 2-wave
# parts; 64 rows of 14 tiles (G=7) become 2-wave parts.
SHAPES = [
    (8, 2, 8, torch.bfloat16),
    (28, 4, 4, torch.bfloat16),
    (8, 2, 8, torch.float32),
]


class _Module(torch.nn.Module):
    layer_idx = 0


def _qkv(seed, B, Hq, Hkv, dtype):
    gen = torch.Generator().manual_seed(seed)
    return [torch.randn(B, T, H, D, generator=gen).to(dtype).to(DEV).transpose(1, 2)
            for H in (Hq, Hkv, Hkv)]


def _rows(rng, B, Hkv, K=6):
    """Causal rows [B, Hkv, QB, K]: the local window (the diagonal and the
    block before it), block 0 and random earlier blocks."""
    idx = np.full((B, Hkv, QB, K), -1, np.int32)
    for b, g, qb in np.ndindex(B, Hkv, QB):
        row = sorted({0, max(0, qb - 1), qb} | set(rng.integers(0, qb + 1, size=K - 3).tolist()))
        idx[b, g, qb, : len(row)] = row
    return idx


def _alone_and_first(call, inputs):
    """call(*inputs) on the first batch element alone and on the whole batch."""
    first = [x[:1] for x in inputs]
    alone = call(*first)
    together = call(*inputs)
    torch.cuda.synchronize()
    return alone, together[:1]


@pytest.mark.parametrize("Hq,Hkv,B,dtype", SHAPES)
@pytest.mark.parametrize("entry", ["index", "key_valid", "attn_mask", "csr", "block_mask",
                                   "summaries", "summaries_key_valid"])
def test_split_and_unsplit_launches_agree(entry, Hq, Hkv, B, dtype):
    print(f"launch shapes: {entry} Hq={Hq} Hkv={Hkv} B={B} {dtype}", flush=True)
    if entry.startswith("summaries") and dtype == torch.float32:
        pytest.skip("summary keys are covered in 16-bit; fp32 runs the same non-producer forms")
    rng = np.random.default_rng(Hq * 100 + B)
    q, k, v = _qkv(Hq + B, B, Hq, Hkv, dtype)
    scale = D ** -0.5
    idx = torch.from_numpy(_rows(rng, B, Hkv)).to(DEV)
    if entry == "index":
        alone, first = _alone_and_first(
            lambda q, k, v, i: direct_index_sparse_prefill(q, k, v, i, scale), (q, k, v, idx))
        expected = ora.sparse_attention_index(*(x[:1].float().cpu().numpy() for x in (q, k, v)),
                                              idx[:1].cpu().numpy())
        err = np.abs(alone.float().cpu().numpy() - expected)
        assert err.max() <= 2e-2 and err.mean() <= 1e-3, (err.max(), err.mean())
    elif entry == "key_valid":
        lengths = torch.tensor(rng.integers(T // 2, T + 1, size=B))
        kv = (torch.arange(T)[None] < lengths[:, None]).to(DEV)
        alone, first = _alone_and_first(
            lambda q, k, v, i, m: direct_index_sparse_prefill(q, k, v, i, scale, key_valid=m),
            (q, k, v, idx, kv))
    elif entry == "attn_mask":
        gen = torch.Generator().manual_seed(7)
        mask = (torch.randn(B, 1, T, T, generator=gen) * 2).to(DEV)
        alone, first = _alone_and_first(
            lambda q, k, v, i, m: direct_index_sparse_prefill(q, k, v, i, scale, attn_mask=m),
            (q, k, v, idx, mask))
    elif entry == "csr":
        lists = idx.reshape(-1, idx.shape[-1]).cpu()
        rows = [r[r >= 0] for r in lists]
        indptr = torch.tensor([0] + np.cumsum([len(r) for r in rows]).tolist(), dtype=torch.int32)
        indices = torch.cat(rows).to(torch.int32)
        n1 = Hkv * QB                                    # the rows of batch element 0
        alone = direct_index_sparse_csr(q[:1], k[:1], v[:1], indptr[: n1 + 1].to(DEV),
                                        indices[: int(indptr[n1])].to(DEV), scale)
        first = direct_index_sparse_csr(q, k, v, indptr.to(DEV), indices.to(DEV), scale)[:1]
    elif entry == "block_mask":
        mask = torch.from_numpy(rng.random((B, Hq, QB, QB)) < 0.3).to(DEV)
        mask |= torch.eye(QB, dtype=torch.bool, device=DEV)
        alone, first = _alone_and_first(lambda q, k, v, m: block_sparse_prefill(q, k, v, m, scale),
                                        (q, k, v, mask))
    elif entry == "summaries_key_valid":
        # The key-padding entry with summaries: the layer's table is built per
        # batch element, so batch element 0's table is the same alone.
        lengths = torch.tensor(rng.integers(T // 2, T + 1, size=B))
        kv = (torch.arange(T)[None] < lengths[:, None]).to(DEV)
        nodes = build_residual_summary_nodes(idx[:, None])[:, 0].to(torch.int32).contiguous()
        lay = build_residual_tree_layout(QB)

        def call(q, k, v, i, n, m):
            table = build_kv_summary_table(k, v, lay, block_size=64, prototypes=2, token_mask=m)
            return direct_index_sparse_summaries(q, k, v, i, n, table, scale, key_valid=m)
        alone, first = _alone_and_first(call, (q, k, v, idx, nodes, kv))
    else:
        selected = idx[:, None]                          # [B, 1, Hkv, QB, K]
        residual = build_residual_summary_nodes(selected)
        assert residual.shape[-1] > 0

        def call(q, k, v, s, r):
            out, _ = sparse_prefill_attention_forward(
                _Module(), q, k, v, None, selected_blocks=s, block_size=64,
                residual_summaries=True, residual_summary_nodes=r, summary_prototypes=2)
            return out
        alone, first = _alone_and_first(call, (q, k, v, selected, residual))
    assert torch.isfinite(alone.float()).all()
    assert torch.equal(alone, first), (entry, (alone.float() - first.float()).abs().max().item())
