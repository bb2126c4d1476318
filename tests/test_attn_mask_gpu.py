"""General 4-D attention masks through the HIP direct-index kernel
(sparse/attention.py:223-229 in the reference: the mask slice at the row's
queries and listed keys is added to the scaled, causally masked scores).

Cases: random additive masks with -inf entries (broadcast and per query
head), packed sequences with a block-diagonal boolean mask, a bf16 padding
mask carrying a score bias, a mask wider than the sequence with
non-multiple-of-4 row strides (element-wise loads), a batch-broadcast mask
(stride 0), float32 inputs, and the producer-wave and 8-wave launch shapes;
masks whose rows are 16-byte aligned (read as row pieces through LDS) in
every element size, with a ragged last block read element-wise.

Bar: 2e-2 max-abs / 1e-3 mean-abs against the float32 oracle
(oracle/attention.py, add_mask) at query rows that keep at least one listed
causal key with a finite mask value (outputs elsewhere are not defined).
"""
import numpy as np
import pytest
import torch

import oracle.attention as ora
from kernels.direct_index import direct_index_sparse_prefill
from sparse.attention import sparse_prefill_attention_forward

pytestmark = pytest.mark.gpu
DEV = "cuda"
MAX_ABS, MEAN_ABS = 2e-2, 1e-3


class _Module(torch.nn.Module):
    layer_idx = 0


def _qkv(seed, B, Hq, Hkv, T, D, dtype):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, Hq, D, generator=gen).to(dtype).transpose(1, 2)
    k = torch.randn(B, T, Hkv, D, generator=gen).to(dtype).transpose(1, 2)
    v = torch.randn(B, T, Hkv, D, generator=gen).to(dtype).transpose(1, 2)
    return q, k, v


def _selection(seed, B, Hkv, T, extra=3):
    Q = (T + 63) // 64
    rng = np.random.default_rng(seed)
    sel = np.full((B, 1, Hkv, Q, extra + 2), -1, np.int32)
    for b, g, qb in np.ndindex(B, Hkv, Q):
        pick = rng.choice(qb + 1, size=min(qb + 1, extra), replace=False).tolist()
        row = sorted(set(pick) | {qb, max(0, qb - 1)})
        sel[b, 0, g, qb, : len(row)] = row
    return torch.from_numpy(sel)


def _dev(*xs):
    return [x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in xs]


def _additive(mask):
    m = mask.cpu()
    if m.dtype == torch.bool:
        return torch.zeros(m.shape).masked_fill(~m, float("-inf")).numpy()
    return m.float().numpy()


def _surviving(sel, mask, Hq):
    """[B, T, Hq]: query rows with at least one listed causal key whose mask
    value is finite.  Other rows are not defined: the kernel writes zeros,
    while the reference's causal fill (finfo.min, not -inf) makes them a
    softmax over the listed future keys, or NaN."""
    idx = sel[:, 0].numpy()
    finite = np.isfinite(_additive(mask))
    B, Hkv, Qb, _ = idx.shape
    T = finite.shape[-1]
    G = Hq // Hkv
    listed = np.zeros((B, Hkv, Qb, Qb), bool)
    for b, g, qb in np.ndindex(B, Hkv, Qb):
        ids = idx[b, g, qb]
        listed[b, g, qb, ids[(ids >= 0) & (ids <= qb)]] = True
    t = np.arange(T)
    keys = np.repeat(listed, 64, axis=-1)[..., :T]                  # [B, Hkv, Qb, T]
    keys = keys[:, :, t // 64] & (t[None, :] <= t[:, None])[None, None]   # [B, Hkv, T, T]
    out = np.zeros((B, T, Hq), bool)
    for h in range(Hq):
        mh = h if finite.shape[1] > 1 else 0
        out[:, :, h] = (keys[:, h // G] & finite[:, mh, :T, :T]).any(-1)
    return out


def _check(out, expected, what, rows=None):
    a = out.float().cpu().numpy().astype(np.float64)
    if rows is None:
        rows = np.isfinite(expected).all(axis=-1)      # [B, T, Hq]
    assert rows.any()
    d = np.abs(a - expected)[rows]
    print(f"{what}: rows={int(rows.sum())}/{rows.size} max_abs={d.max():.3e} mean_abs={d.mean():.3e}",
          flush=True)
    assert np.isfinite(a[rows]).all()
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, (what, d.max(), d.mean())


def _oracle(q, k, v, sel, mask):
    return ora.sparse_attention_index(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                      sel[:, 0].numpy(), add_mask=_additive(mask))


@pytest.mark.parametrize("Hq,Hkv,T,D,dtype,Hm", [
    (28, 4, 700, 128, torch.bfloat16, 1),    # Qwen2-7B heads, producer-wave form
    (28, 4, 700, 128, torch.bfloat16, 28),   # one mask per query head
    (8, 2, 333, 64, torch.float16, 8),       # G=4, full 8-wave parts
    (6, 2, 260, 128, torch.float32, 1),      # 16-byte rows: row pieces, last block element-wise
    (28, 4, 512, 128, torch.bfloat16, 28),   # 16-byte rows, per head, producer form
    (8, 2, 448, 64, torch.float16, 1),       # 16-byte rows, 8-wave parts
])
def test_random_additive_mask_matches_oracle(Hq, Hkv, T, D, dtype, Hm):
    seed = T + Hq + Hm
    q, k, v = _qkv(seed, 2, Hq, Hkv, T, D, dtype)
    sel = _selection(seed, 2, Hkv, T)
    gen = torch.Generator().manual_seed(seed + 1)
    mask = torch.randn(2, Hm, T, T, generator=gen) * 3
    mask[torch.rand(mask.shape, generator=gen) < 0.2] = float("-inf")
    mask = mask.to(dtype)
    qd, kd, vd = _dev(q, k, v)
    out, _ = sparse_prefill_attention_forward(
        _Module(), qd, kd, vd, mask.to(DEV), selected_blocks=sel.to(DEV), block_size=64,
        validate_selected_blocks_input=False)
    torch.cuda.synchronize()
    _check(out, _oracle(q, k, v, sel, mask), f"additive Hq{Hq} Hkv{Hkv} T{T} D{D} {dtype} Hm{Hm}",
           _surviving(sel, mask, Hq))
    direct = direct_index_sparse_prefill(qd, kd, vd, sel[:, 0].contiguous().to(DEV), scale=D ** -0.5,
                                         attn_mask=mask.to(DEV))
    assert torch.equal(direct, out)


def test_packed_sequences_with_a_block_diagonal_bool_mask():
    # Three sequences packed into one row of 640 tokens (starts 0, 200, 450),
    # the mask Transformers builds for packed inputs: attend where both tokens
    # are in the same sequence and the key is not in the future.
    T, Hq, Hkv, D = 640, 28, 4, 128
    q, k, v = _qkv(21, 1, Hq, Hkv, T, D, torch.bfloat16)
    sel = _selection(21, 1, Hkv, T, extra=10)
    seg = torch.zeros(T, dtype=torch.long)
    seg[200:] = 1
    seg[450:] = 2
    causal = torch.tril(torch.ones(T, T, dtype=torch.bool))
    mask = (causal & (seg[:, None] == seg[None, :]))[None, None]
    qd, kd, vd = _dev(q, k, v)
    out, _ = sparse_prefill_attention_forward(
        _Module(), qd, kd, vd, mask.to(DEV), selected_blocks=sel.to(DEV), block_size=64,
        validate_selected_blocks_input=False)
    torch.cuda.synchronize()
    expected = _oracle(q, k, v, sel, mask)
    _check(out, expected, "packed bool", _surviving(sel, mask, Hq))
    # With every causal block listed, each sequence equals its attention alone.
    Q = (T + 63) // 64
    full = torch.full((1, 1, Hkv, Q, Q), -1, dtype=torch.int32)
    for qb in range(Q):
        full[..., qb, : qb + 1] = torch.arange(qb + 1, dtype=torch.int32)
    out_full, _ = sparse_prefill_attention_forward(
        _Module(), qd, kd, vd, mask.to(DEV), selected_blocks=full.to(DEV), block_size=64,
        validate_selected_blocks_input=False)
    torch.cuda.synchronize()
    a = out_full.float().cpu().numpy()
    for s0, s1 in ((0, 200), (200, 450), (450, 640)):
        alone = ora.dense_causal_attention(q[:, :, s0:s1].float().numpy(), k[:, :, s0:s1].float().numpy(),
                                           v[:, :, s0:s1].float().numpy())
        d = np.abs(a[:, s0:s1] - alone)
        assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, (s0, d.max(), d.mean())


def test_bf16_padding_mask_with_a_score_bias():
    # The eager-path mask layout (0 / finfo.min) with a bias on some keys:
    # no longer key padding, so the kernel reads the mask itself.
    T, Hq, Hkv, D = 500, 28, 4, 128
    q, k, v = _qkv(31, 2, Hq, Hkv, T, D, torch.bfloat16)
    sel = _selection(31, 2, Hkv, T)
    valid = torch.zeros(2, T, dtype=torch.bool)
    valid[0, :420] = True
    valid[1, 90:] = True
    allowed = torch.tril(torch.ones(T, T, dtype=torch.bool))[None] & valid[:, None, :]
    mask = torch.zeros(2, 1, T, T, dtype=torch.bfloat16)
    mask.masked_fill_(~allowed[:, None], torch.finfo(torch.bfloat16).min)
    mask[:, :, :, 64:80] += -1.5
    qd, kd, vd = _dev(q, k, v)
    out, _ = sparse_prefill_attention_forward(
        _Module(), qd, kd, vd, mask.to(DEV), selected_blocks=sel.to(DEV), block_size=64,
        validate_selected_blocks_input=False)
    torch.cuda.synchronize()
    expected = _oracle(q, k, v, sel, mask)
    rows = _surviving(sel, torch.where(mask.float() > -1e30, 0.0, float("-inf")), Hq)
    rows &= valid.numpy()[:, :, None]              # padding query positions are not defined
    _check(out, expected, "bf16 padding + bias", rows)
    # Without the bias the same mask is key padding: both kernels agree.
    plain = torch.zeros(2, 1, T, T, dtype=torch.bfloat16).masked_fill_(
        ~allowed[:, None], torch.finfo(torch.bfloat16).min).to(DEV)
    by_valid = direct_index_sparse_prefill(qd, kd, vd, sel[:, 0].contiguous().to(DEV), scale=D ** -0.5,
                                           key_valid=valid.to(DEV))
    by_mask = direct_index_sparse_prefill(qd, kd, vd, sel[:, 0].contiguous().to(DEV), scale=D ** -0.5,
                                          attn_mask=plain)
    torch.cuda.synchronize()
    d = (by_valid.float() - by_mask.float()).abs()[valid.to(DEV)]
    assert d.max().item() <= 1e-2, d.max().item()


@pytest.mark.parametrize("layout", ["wide", "broadcast"])
def test_mask_layouts(layout):
    # "wide": a [B, Hq, T + 3, T + 5] float32 mask sliced by the kernel (row
    # strides not multiples of 4, so element-wise loads); "broadcast": one
    # float16 mask expanded over the batch (stride 0).
    T, Hq, Hkv, D = 390, 8, 2, 128
    q, k, v = _qkv(41, 2, Hq, Hkv, T, D, torch.bfloat16)
    sel = _selection(41, 2, Hkv, T)
    gen = torch.Generator().manual_seed(42)
    if layout == "wide":
        big = torch.randn(2, Hq, T + 3, T + 5, generator=gen)
        big[torch.rand(big.shape, generator=gen) < 0.1] = float("-inf")
        mask_dev = big.to(DEV)
        mask_ref = big[:, :, :T, :T]
    else:
        one = (torch.randn(1, 1, T, T, generator=gen) * 2).half()
        mask_dev = one.to(DEV).expand(2, 1, T, T)
        mask_ref = one.expand(2, 1, T, T)
    qd, kd, vd = _dev(q, k, v)
    out = direct_index_sparse_prefill(qd, kd, vd, sel[:, 0].contiguous().to(DEV), scale=D ** -0.5,
                                      attn_mask=mask_dev)
    torch.cuda.synchronize()
    _check(out, _oracle(q, k, v, sel, mask_ref), f"layout {layout}", _surviving(sel, mask_ref, Hq))


def test_zero_mask_equals_no_mask_and_residual_summaries_reject_other_masks():
    T, Hq, Hkv, D = 300, 28, 4, 128
    q, k, v = _qkv(51, 1, Hq, Hkv, T, D, torch.bfloat16)
    sel = _selection(51, 1, Hkv, T)
    qd, kd, vd = _dev(q, k, v)
    idx = sel[:, 0].contiguous().to(DEV)
    zero = torch.zeros(1, 1, T, T, device=DEV)
    a = direct_index_sparse_prefill(qd, kd, vd, idx, scale=D ** -0.5, attn_mask=zero)
    b = direct_index_sparse_prefill(qd, kd, vd, idx, scale=D ** -0.5)
    torch.cuda.synchronize()
    assert (a.float() - b.float()).abs().max().item() <= 1e-2
    bias = torch.randn(1, 1, T, T, device=DEV)
    nodes = torch.full(sel.shape[:4] + (2,), -1, dtype=torch.int32)
    with pytest.raises(ValueError, match="another pattern"):
        sparse_prefill_attention_forward(
            _Module(), qd, kd, vd, bias, selected_blocks=sel.to(DEV), block_size=64,
            validate_selected_blocks_input=False, residual_summaries=True,
            residual_summary_nodes=nodes.to(DEV), validate_residual_summary_nodes_input=False)


@pytest.mark.parametrize("Hm", [1, 8])
def test_bool_mask_in_16_byte_rows(Hm):
    # T = 320: a bool row is 320 bytes, so blocks are read as row pieces.
    T, Hq, Hkv, D = 320, 8, 2, 128
    q, k, v = _qkv(61 + Hm, 2, Hq, Hkv, T, D, torch.bfloat16)
    sel = _selection(61 + Hm, 2, Hkv, T)
    gen = torch.Generator().manual_seed(62 + Hm)
    mask = torch.rand(2, Hm, T, T, generator=gen) < 0.8
    qd, kd, vd = _dev(q, k, v)
    out = direct_index_sparse_prefill(qd, kd, vd, sel[:, 0].contiguous().to(DEV), scale=D ** -0.5,
                                      attn_mask=mask.to(DEV))
    torch.cuda.synchronize()
    _check(out, _oracle(q, k, v, sel, mask), f"bool rows Hm{Hm}", _surviving(sel, mask, Hq))
