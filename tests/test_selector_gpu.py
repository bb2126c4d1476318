"""Selector kernels (through the C ABI) against the C oracle, bit for bit.

Pooled summaries, projections, scores and the selected block indices must be
identical to oracle/selector.c (the same IEEE float32 operation order); the
full cfg3 workload (T=65536, 28/4 heads, d=128, top-32) is checked end to end.
"""
import numpy as np
import pytest
import torch

import oracle.selector as osel
from selector.gate import FlatGate
from selector.select import causal_topk_blocks, gate_scores, pool_blocks, project, project_pair, select_blocks
from spruce_hip import workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("B,Hq,Hkv,T,D,dtype", [
    (1, 28, 4, 1000, 128, torch.bfloat16),
    (2, 8, 2, 200, 64, torch.float16),
    (1, 4, 4, 64, 128, torch.float32),
    (1, 12, 2, 129, 16, torch.bfloat16),
    (1, 16, 2, 300, 256, torch.bfloat16),   # G = 8, 8 token steps per thread: the typed kernel's limits
    (1, 18, 2, 150, 128, torch.float16),    # G = 9: the generic kernel
    (1, 4, 2, 100, 512, torch.float32),     # 16 token steps per thread: the generic kernel
    (1, 12, 2, 150, 96, torch.bfloat16),    # 16 lanes of 12 dim chunks: head_dim not a power of two
    (1, 8, 4, 129, 80, torch.float16),
    (1, 4, 1, 70, 2040, torch.float32),     # one lane of 255 dim chunks, 64 token steps
])
def test_pooling_is_bit_exact(B, Hq, Hkv, T, D, dtype):
    gen = torch.Generator().manual_seed(T + D)
    q = torch.randn(B, T, Hq, D, generator=gen).to(dtype).transpose(1, 2)   # strided view
    k = torch.randn(B, Hkv, T, D, generator=gen).to(dtype)
    qm, ks = pool_blocks(q.transpose(1, 2).contiguous().to(DEV).transpose(1, 2), k.to(DEV))
    eqm, eks = osel.block_pool(q.float().numpy(), k.float().numpy())
    assert np.array_equal(_np(qm), eqm)
    assert np.array_equal(_np(ks), eks)
    # Every token of every block is pooled: float64 block means and exact maxima.
    nb = (T + 63) // 64
    q64 = q.double().reshape(B, Hkv, Hq // Hkv, T, D).mean(dim=2)
    for blk in range(nb):
        sl = slice(64 * blk, min(T, 64 * blk + 64))
        np.testing.assert_allclose(_np(qm[:, :, blk]), q64[:, :, sl].mean(dim=2).numpy(), rtol=0, atol=5e-6)
        np.testing.assert_allclose(_np(ks[:, :, blk, 0]), k[:, :, sl].double().mean(dim=2).numpy(),
                                   rtol=0, atol=5e-6)
        assert torch.equal(ks[:, :, blk, 1].cpu(), k[:, :, sl].float().amax(dim=2))
    _, ks_only = pool_blocks(None, k.to(DEV))
    assert torch.equal(ks_only, ks)


def test_projection_scores_and_topk_are_bit_exact():
    gen = torch.Generator().manual_seed(7)
    S, Qb, Pq, Pk, D, P = 3, 77, 2, 3, 96, 64
    qf = torch.randn(S, Qb, Pq, D, generator=gen)
    kf = torch.randn(S, Qb, Pk, D, generator=gen)
    Wq = torch.randn(D, P, generator=gen) * 0.1
    Wk = torch.randn(D, P, generator=gen) * 0.1
    qp, kp = project(qf.to(DEV), Wq), project(kf.to(DEV), Wk)
    eqp, ekp = osel.project(qf.numpy(), Wq.numpy()), osel.project(kf.numpy(), Wk.numpy())
    assert np.array_equal(_np(qp), eqp) and np.array_equal(_np(kp), ekp)
    for causal in (True, False):
        s = gate_scores(qp, kp, causal=causal)
        es = osel.scores(eqp, ekp, causal=causal)
        assert np.array_equal(_np(s), es), causal
    sel = causal_topk_blocks(gate_scores(qp, kp), 5)
    assert np.array_equal(_np(sel), osel.topk(osel.scores(eqp, ekp), 5))


@pytest.mark.parametrize("N,D,P", [(1, 4, 4), (65, 96, 36), (200, 256, 128), (130, 160, 68), (33, 6, 5),
                                   (4096 * 8, 128, 128), (16384 + 77, 100, 68), (20000, 260, 36)])
def test_projection_shapes_are_bit_exact(N, D, P):
    # Vector tiles (D % 4 == 0, P % 4 == 0: ragged rows and columns, two
    # 128-wide slices of D), the scalar form (D = 6, P = 5) and, from 16K
    # rows, 8 x 4 register tiles (ragged last row tile, D not a multiple of
    # the 32-dim slice, P not a multiple of the 64-column tile).
    gen = torch.Generator().manual_seed(N + D + P)
    x = torch.randn(N, D, generator=gen)
    W = torch.randn(D, P, generator=gen) * 0.1
    got = project(x.to(DEV), W)
    assert np.array_equal(_np(got), osel.project(x.numpy(), W.numpy()))


@pytest.mark.parametrize("Na,Nb,D,P", [
    (4096, 8192, 128, 128),   # cfg3: query and key prototypes of 4 KV heads x 1024 blocks
    (77, 130, 96, 36),        # ragged 32-row tiles and 64-column tiles
    (1, 33, 128, 64),
    (5, 7, 6, 5),             # scalar form: two launches
    (20000, 100, 128, 128),   # block kernel for the large side: two launches
])
def test_projection_pair_equals_single_launches(Na, Nb, D, P):
    gen = torch.Generator().manual_seed(Na + Nb + D)
    xa, xb = torch.randn(Na, D, generator=gen), torch.randn(Nb, D, generator=gen)
    Wa, Wb = torch.randn(D, P, generator=gen) * 0.1, torch.randn(D, P, generator=gen) * 0.1
    oa, ob = project_pair(xa.to(DEV), Wa.to(DEV), xb.to(DEV), Wb.to(DEV))
    assert np.array_equal(_np(oa), osel.project(xa.numpy(), Wa.numpy()))
    assert np.array_equal(_np(ob), osel.project(xb.numpy(), Wb.numpy()))
    assert torch.equal(oa, project(xa.to(DEV), Wa)) and torch.equal(ob, project(xb.to(DEV), Wb))


@pytest.mark.parametrize("dtype,S,nodes,Pk,D,P", [
    (torch.bfloat16, 4, [2048, 1024, 512, 256, 128, 64, 32, 16, 8, 4, 2, 1], 8, 128, 128),  # cfg5 key tree
    (torch.float16, 3, [37, 19, 10, 5, 3, 2, 1], 4, 64, 36),   # ragged tiles, levels smaller than a tile
    (torch.float32, 2, [100], 2, 96, 128),                      # one level (the query prototypes' use)
    (torch.bfloat16, 1, [1, 1, 1], 1, 8, 4),                    # tiny levels and dims
])
def test_projection_of_levels_equals_projection_of_their_float_copy(dtype, S, nodes, Pk, D, P):
    # spruce_gate_project_levels reads each level in the model dtype and
    # widens it exactly: bit-identical to projecting a float32 copy of the
    # concatenated levels, which the oracle pins.
    from selector.select import project_levels
    gen = torch.Generator().manual_seed(S + D + P + len(nodes))
    levels = [torch.randn(S, n, Pk, D, generator=gen).to(dtype) for n in nodes]
    W = torch.randn(D, P, generator=gen) * 0.1
    got = project_levels([t.to(DEV) for t in levels], W.to(DEV))
    flat = torch.cat(levels, dim=1).float()
    assert got.shape == (S, sum(nodes), Pk, P)
    assert torch.equal(got, project(flat.to(DEV), W))
    # The interleaved layout holds the same values: [S, N, P/4, Pk, 4].
    il = project_levels([t.to(DEV) for t in levels], W.to(DEV), interleaved=True)
    assert il.shape == (S, sum(nodes), P // 4, Pk, 4)
    assert torch.equal(il, got.reshape(S, sum(nodes), Pk, P // 4, 4).transpose(2, 3))
    if flat.numel() * P <= 1 << 24:
        assert np.array_equal(_np(got).reshape(-1, P), osel.project(flat.reshape(-1, D).numpy(), W.numpy()))


def test_flat_gate_key_levels_and_model_dtype_queries():
    gen = torch.Generator().manual_seed(11)
    gate = FlatGate(2, 64, proj_dim=32).to(DEV).eval()
    q = torch.randn(2, 3, 40, 4, 64, generator=gen).to(torch.bfloat16).to(DEV)
    levels = [torch.randn(2, 3, n, 4, 64, generator=gen).to(torch.bfloat16).to(DEV) for n in (40, 20, 10, 5, 3, 2, 1)]
    with torch.no_grad():
        rows = gate.project_keys(torch.cat(levels, dim=2).float())
        assert torch.equal(gate.project_key_levels(levels), rows)
        il = rows.reshape(2, 3, 81, 4, 8, 4).transpose(3, 4)
        assert torch.equal(gate.project_key_levels(levels, interleaved=True), il)
        # Features the kernel does not read directly (float64) take project_keys, then the same layout.
        assert torch.equal(gate.project_key_levels([x.double() for x in levels], interleaved=True), il)
        assert torch.equal(gate.project_queries(q), gate.project_queries(q.float()))


@pytest.mark.parametrize("S,Qb,Pk,P", [
    (2, 130, 2, 128),    # triangular tile grid, ragged last tile
    (4, 1024, 2, 128),   # cfg3 score shape
    (1, 64, 1, 64),
    (1, 1, 2, 128),
    (1, 200, 2, 48),     # P % 32 != 0: the broadcast kernel (full -inf fill)
])
def test_lower_scores_equal_the_causal_fill_on_and_below_the_diagonal(S, Qb, Pk, P):
    # causal="lower" launches only the tiles on or below the diagonal; the
    # causal entries must equal the fully filled causal matrix bit for bit.
    gen = torch.Generator().manual_seed(Qb + P)
    qp = torch.randn(S, Qb, 1, P, generator=gen).to(DEV)
    kp = torch.randn(S, Qb, Pk, P, generator=gen).to(DEV)
    full = gate_scores(qp, kp, causal=True)
    lower = gate_scores(qp, kp, causal="lower")
    tril = torch.tril(torch.ones(Qb, Qb, dtype=torch.bool, device=DEV))
    assert torch.equal(full[:, tril], lower[:, tril])
    assert torch.equal(causal_topk_blocks(lower, 16), causal_topk_blocks(full, 16))


@pytest.mark.parametrize("S,Qb,Kb,Pk,P", [
    (2, 130, 130, 2, 128),   # register-blocked tiles: ragged last tile row and column
    (1, 77, 190, 1, 64),     # one key prototype, Qb != Kb
    (3, 64, 67, 2, 32),      # Kb % 4 != 0: scalar stores at the row ends
    (1, 200, 200, 2, 48),    # P % 32 != 0: the LDS-broadcast tile kernel
    (1, 1, 1, 2, 128),
])
def test_score_tile_shapes_are_bit_exact(S, Qb, Kb, Pk, P):
    gen = torch.Generator().manual_seed(Qb * 7 + Kb + P)
    qp = torch.randn(S, Qb, 1, P, generator=gen)
    kp = torch.randn(S, Kb, Pk, P, generator=gen)
    for causal in (True, False):
        got = gate_scores(qp.to(DEV), kp.to(DEV), causal=causal)
        assert np.array_equal(_np(got), osel.scores(qp.numpy(), kp.numpy(), causal=causal)), causal


def test_scores_with_eight_prototypes_per_side_are_bit_exact():
    # The reference's captured features carry 8 prototypes per block on each
    # side; their tiles exceed LDS, so the direct kernel computes them.
    gen = torch.Generator().manual_seed(13)
    S, Qb, Pq, Pk, P = 2, 45, 8, 8, 128
    qp = torch.randn(S, Qb, Pq, P, generator=gen)
    kp = torch.randn(S, Qb, Pk, P, generator=gen)
    for causal in (True, False):
        got = gate_scores(qp.to(DEV), kp.to(DEV), causal=causal)
        assert np.array_equal(_np(got), osel.scores(qp.numpy(), kp.numpy(), causal=causal)), causal
    sel = causal_topk_blocks(gate_scores(qp.to(DEV), kp.to(DEV)), 8)
    assert np.array_equal(_np(sel), osel.topk(osel.scores(qp.numpy(), kp.numpy()), 8))


def test_topk_ties_short_rows_and_negative_zero():
    gen = torch.Generator().manual_seed(11)
    s = torch.randn(2, 300, 300, generator=gen)
    s[0, 250, :251] = 1.5                      # all tied: lowest indices win
    s[0, 120, [4, 50, 99, 100]] = 9.0          # tie at the top
    s[1, 200, :201] = 0.0
    s[1, 200, ::2] = -0.0                      # +0 / -0 tie, treated as equal
    s[1, 280, 17] = float("inf")
    got = causal_topk_blocks(s.to(DEV), 32)
    exp = osel.topk(s.numpy(), 32)
    assert np.array_equal(_np(got), exp)
    assert _np(got)[0, 250].tolist() == list(range(32))
    assert _np(got)[0, 10].tolist() == list(range(11)) + [-1] * 21


def test_topk_search_boundaries():
    # Rows with heavy ties, a one-ulp gap at the k-th key, exactly k tied top
    # keys, a tie across the boundary and full 1024-key rows.
    gen = torch.Generator().manual_seed(5)
    s = torch.randn(3, 1024, 1024, generator=gen)
    s[1] = torch.round(s[1] * 4) / 4
    row = s[2, 700, :701]
    order = torch.argsort(row, descending=True, stable=True)
    kth = row[order[31]].item()
    s[2, 700, order[32]] = float(np.nextafter(np.float32(kth), np.float32(-np.inf)))
    s[2, 800, torch.randperm(801, generator=gen)[:32]] = 5.0
    s[2, 900, torch.randperm(901, generator=gen)[:33]] = 5.0     # the tie crosses the boundary
    got = causal_topk_blocks(s.to(DEV), 32)
    assert np.array_equal(_np(got), osel.topk(s.numpy(), 32))


@pytest.mark.parametrize("k", [32, 100])
def test_topk_rows_longer_than_1024_blocks(k):
    # Rows of more than 1024 key blocks take the LDS radix-select kernel.
    gen = torch.Generator().manual_seed(13)
    s = torch.randn(2, 1500, 1500, generator=gen)
    s[0, 1400, :1401] = torch.round(s[0, 1400, :1401] * 2) / 2    # heavy ties
    s[0, 1300, torch.randperm(1301, generator=gen)[:40]] = 7.0    # a tie across the top-32 boundary
    s[1, 1499, :1500] = 0.0
    s[1, 1499, ::3] = -0.0                                         # +0 / -0 tie, treated as equal
    got = causal_topk_blocks(s.to(DEV), k)
    assert np.array_equal(_np(got), osel.topk(s.numpy(), k))


@pytest.mark.parametrize("k", [1, 8, 32, 64, 65])
def test_topk_candidate_search_and_its_fallback(k):
    # The top-k search first bounds the k-th key by the k-th largest lane
    # maximum and searches among the (at most 64) keys above that bound;
    # rows with more than 64 such keys (heavy ties, few distinct values) and
    # k > 64 take the full search.  Both must give the oracle's indices.
    gen = torch.Generator().manual_seed(23)
    s = torch.randn(4, 1024, 1024, generator=gen)            # distinct keys: the candidate search
    s[1] = torch.randint(0, 3, (1024, 1024), generator=gen).float()   # three values: the fallback
    s[2, :, :] = 0.25                                         # one value everywhere
    s[3] = torch.randint(0, 40, (1024, 1024), generator=gen).float() * 0.5
    s[3, 600, :601] = torch.arange(601, dtype=torch.float32).flip(0)  # strictly decreasing row
    s[3, 601, 7::64] = 50.0                                   # the top keys all in one lane
    got = causal_topk_blocks(s.to(DEV), k)
    assert np.array_equal(_np(got), osel.topk(s.numpy(), k))


def test_flat_gate_matches_reference_bruteforce():
    # Reference tests/test_gate_maxsim.py:22-33 on the HIP scorer.
    torch.manual_seed(0)
    L, G, qb, kb, P, d = 2, 2, 3, 3, 4, 8
    gate = FlatGate(L, d, proj_dim=d).eval()
    q = torch.randn(L, G, qb, P, d)
    k = torch.randn(L, G, kb, P, d)
    with torch.no_grad():
        s = gate.to(DEV)(q.to(DEV), k.to(DEV))
        qp = torch.einsum("lgqid,ldp->lgqip", q.double(), gate.Wq.cpu().double())
        kp = torch.einsum("lgkjd,ldp->lgkjp", k.double(), gate.Wk.cpu().double())
        ref = torch.einsum("lgqip,lgkjp->lgqkij", qp, kp).amax(dim=(-1, -2)) / gate.proj_dim ** 0.5
    assert s.shape == (L, G, qb, kb)
    torch.testing.assert_close(s.cpu().double(), ref, atol=1e-5, rtol=1e-5)
    with pytest.raises(RuntimeError, match="no_grad"):
        gate(q.to(DEV), k.to(DEV))


def test_cfg3_full_size_selected_blocks_bit_exact():
    # Benchmark configuration cfg3: T=65536 (1024 key blocks), 28 Q / 4 KV heads, d=128, bf16, top-32.
    print("cfg3: generating inputs", flush=True)
    q, k, _ = workloads.qkv(0, 65536, 28, 4, 128, torch.bfloat16, use_rope=False, layout="bthd")
    Wq, Wk = workloads.cfg3_gate_weights(0)
    got = select_blocks(q.transpose(1, 2).contiguous().to(DEV).transpose(1, 2), k.to(DEV),
                        Wq.to(DEV), Wk.to(DEV), top_k=32, return_intermediates=True)
    torch.cuda.synchronize()
    print("cfg3: oracle", flush=True)
    exp = osel.flat_select(q.float().numpy(), k.float().numpy(), Wq.numpy(), Wk.numpy(), top_k=32)
    for name in ("q_mean", "k_sum", "scores"):
        assert np.array_equal(_np(got[name]), exp[name]), name
    assert np.array_equal(_np(got["qp"]), exp["qp"][:, :, :, 0])
    assert np.array_equal(_np(got["kp"]), exp["kp"])
    sel = _np(got["selected"])
    assert sel.shape == (1, 1, 4, 1024, 32) and sel.dtype == np.int32
    assert np.array_equal(sel, exp["selected"])
    # Contract: causal, strictly increasing, trailing -1 padding, full rows after block 31.
    rows = sel[0, 0].reshape(-1, 32)
    valid = rows >= 0
    assert np.all(rows[valid] <= np.repeat(np.arange(1024)[None], 4, 0).reshape(-1, 1).repeat(32, 1)[valid])
    both = valid[:, 1:] & valid[:, :-1]
    assert np.all(np.diff(rows, axis=1)[both] > 0)              # strictly increasing
    assert np.all(~valid[:, 1:] | valid[:, :-1])                # padding only trailing
    assert valid.reshape(4, 1024, 32)[:, 31:].all()             # >= 32 causal blocks: full rows
    # The production path (paired projection, scores on and below the diagonal only).
    fast = select_blocks(q.transpose(1, 2).contiguous().to(DEV).transpose(1, 2), k.to(DEV),
                         Wq.to(DEV), Wk.to(DEV), top_k=32)
    assert np.array_equal(_np(fast), exp["selected"])
    # The two-launch fused route at full size.
    from selector.select import select_blocks_fused
    fused = select_blocks_fused(q.transpose(1, 2).contiguous().to(DEV).transpose(1, 2), k.to(DEV),
                                Wq.to(DEV), Wk.to(DEV), top_k=32)
    assert np.array_equal(_np(fused), exp["selected"])


# The fused route (key side in one launch, one persistent launch that pools
# and projects the next tile of query blocks while the current one is scored
# and selected) against the four-launch route and the oracle.  Cases: every query
# heads per KV head from 1 to 8, ragged T (partial last block, partial last
# tile of 4 blocks), B > 1, both 16-bit dtypes, strided [B, T, H, D] storage,
# k = 1, k above 64 (the top-k's full search) and k above the block count, and
# the 1024-block maximum.
@pytest.mark.parametrize("B,Hq,Hkv,T,k,dtype,bthd", [
    (2, 8, 2, 1000, 32, torch.bfloat16, True),
    (1, 7, 1, 64, 8, torch.float16, False),
    (1, 8, 1, 5000, 64, torch.bfloat16, True),
    (3, 3, 3, 777, 5, torch.float16, False),
    (1, 10, 2, 4113, 33, torch.bfloat16, False),
    (1, 6, 2, 65536, 100, torch.bfloat16, True),
    (1, 2, 1, 130, 200, torch.float16, True),
    (2, 12, 2, 3000, 1, torch.bfloat16, True),
    (1, 14, 2, 1601, 16, torch.float16, True),
])
def test_fused_route_equals_four_launch_route(B, Hq, Hkv, T, k, dtype, bthd):
    from selector.select import fused_route_applies, select_blocks_fused
    D = P = 128
    print(f"fused selector B={B} Hq={Hq} Hkv={Hkv} T={T} k={k} {dtype}", flush=True)
    gen = torch.Generator().manual_seed(T + Hq + k)
    if bthd:
        q = torch.randn(B, T, Hq, D, generator=gen).to(dtype).to(DEV).transpose(1, 2)
    else:
        q = torch.randn(B, Hq, T, D, generator=gen).to(dtype).to(DEV)
    kk = torch.randn(B, Hkv, T, D, generator=gen).to(dtype).to(DEV)
    Wq = (torch.randn(D, P, generator=gen) / D ** 0.5).to(DEV)
    Wk = (torch.randn(D, P, generator=gen) / D ** 0.5).to(DEV)
    assert fused_route_applies(q, kk, Wq, Wk)
    fused = select_blocks_fused(q, kk, Wq, Wk, top_k=k)
    four = select_blocks(q, kk, Wq, Wk, top_k=k, return_intermediates=True)["selected"]
    torch.cuda.synchronize()
    assert fused.shape == four.shape == (B, 1, Hkv, (T + 63) // 64, k)
    assert torch.equal(fused, four)
    assert torch.equal(select_blocks(q, kk, Wq, Wk, top_k=k), fused)   # the default (four-launch) route
    if T <= 5000:
        exp = osel.flat_select(q.float().cpu().numpy(), kk.float().cpu().numpy(), Wq.cpu().numpy(),
                               Wk.cpu().numpy(), top_k=k)
        assert np.array_equal(_np(fused), exp["selected"])


def test_fused_route_applies_only_to_its_shapes():
    from selector.select import fused_route_applies
    W = torch.zeros(128, 128, device=DEV)
    q = torch.zeros(1, 8, 256, 128, device=DEV, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 256, 128, device=DEV, dtype=torch.bfloat16)
    assert fused_route_applies(q, k, W, W)
    assert not fused_route_applies(q.float(), k.float(), W, W)                        # float32 inputs
    assert not fused_route_applies(q[..., :64], k[..., :64], W[:64], W[:64])          # head_dim 64
    assert not fused_route_applies(q, k, W[:, :64], W[:, :64])                         # projection dim 64
    assert not fused_route_applies(torch.zeros(1, 18, 256, 128, device=DEV, dtype=torch.bfloat16), k, W, W)  # G 9
    long_q = torch.zeros(1, 2, 1024 * 64 + 1, 128, device=DEV, dtype=torch.bfloat16)   # 1025 key blocks
    assert not fused_route_applies(long_q, long_q[:, :1], W, W)


# Pooling + projection in one launch against the two launches it replaces,
# bit for bit: every query heads per KV head from 1 to 8, ragged T, B > 1,
# both 16-bit dtypes, [B, T, H, D] and [B, H, T, D] storage.
@pytest.mark.parametrize("B,Hq,Hkv,T,dtype,bthd", [
    (1, 28, 4, 4097, torch.bfloat16, True),
    (2, 8, 2, 1000, torch.float16, False),
    (1, 8, 1, 130, torch.bfloat16, True),
    (3, 3, 3, 64, torch.float16, True),
    (1, 10, 2, 70000, torch.bfloat16, False),   # more than 1024 blocks
    (1, 12, 2, 77, torch.bfloat16, True),
    (1, 4, 4, 3333, torch.float16, True),
    (1, 6, 1, 640, torch.bfloat16, False),
])
def test_pool_project_equals_pool_then_project(B, Hq, Hkv, T, dtype, bthd):
    from selector.select import pool_project, pool_project_applies
    D = P = 128
    print(f"pool_project B={B} Hq={Hq} Hkv={Hkv} T={T} {dtype}", flush=True)
    gen = torch.Generator().manual_seed(T + Hq)
    if bthd:
        q = torch.randn(B, T, Hq, D, generator=gen).to(dtype).to(DEV).transpose(1, 2)
        kk = torch.randn(B, T, Hkv, D, generator=gen).to(dtype).to(DEV).transpose(1, 2)
    else:
        q = torch.randn(B, Hq, T, D, generator=gen).to(dtype).to(DEV)
        kk = torch.randn(B, Hkv, T, D, generator=gen).to(dtype).to(DEV)
    Wq = (torch.randn(D, P, generator=gen) / D ** 0.5).to(DEV)
    Wk = (torch.randn(D, P, generator=gen) / D ** 0.5).to(DEV)
    assert pool_project_applies(q, kk, Wq, Wk)
    qp, kp = pool_project(q, kk, Wq, Wk)
    qm, ks = pool_blocks(q, kk)
    eqp, ekp = project_pair(qm, Wq, ks, Wk)
    torch.cuda.synchronize()
    assert torch.equal(qp, eqp)
    assert torch.equal(kp, ekp)
    if T <= 1000:
        exp = osel.flat_select(q.float().cpu().numpy(), kk.float().cpu().numpy(), Wq.cpu().numpy(),
                               Wk.cpu().numpy(), top_k=8)
        assert np.array_equal(_np(select_blocks(q, kk, Wq, Wk, top_k=8)), exp["selected"])
