"""Selector prototype features (HIP, through the C ABI) against the oracle.

Bar: bit-exact (same float32 operation order and model-dtype rounding as
oracle/proto.c).  Cases: the reference's own known answers (needle kept in
fp32/fp16/bf16, ragged block padded with the mean), query-side group averaging
(28 query heads over 4 KV groups) and key-side pooling (no averaging), all
three dtypes, strided query views ([B,T,H,D] storage as the HF hook passes
it), head_dim 4 (the scalar path), block < 64 and P > block + 1.  Full size
(the cfg3 shapes, T = 65536): every block of one KV group against the oracle,
plus mean-prototype invariants over all groups.
"""
import numpy as np
import pytest
import torch

import oracle.selector as osel
from spruce_hip import workloads
from teacher.chunked_extract import _group_avg_tokens, _proto_pool_seq, proto_pool_grouped

pytestmark = pytest.mark.gpu
DEV = "cuda"
_NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


def _oracle(x, G, block, P):
    name = _NAMES[x.dtype]
    a = x.float().cpu().numpy()
    if G != x.shape[1]:
        a = osel.group_avg(a, G, name)
    return osel.proto_pool(a, block, P, name)


def _same(got, exp, what):
    g = got.float().cpu().numpy()
    bad = np.argwhere(~((g == exp) | (np.isnan(g) & np.isnan(exp))))
    assert bad.size == 0, (what, bad[:5].tolist(), g[tuple(bad[0])], exp[tuple(bad[0])])


def test_reference_known_answers():
    torch.manual_seed(0)
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        x = (torch.randn(1, 1, 64, 128) * 0.01).to(dtype)
        x[0, 0, 37, :] = 40.0
        out = _proto_pool_seq(x.to(DEV), 64, 8).cpu()
        assert out.dtype == dtype and out.shape == (1, 1, 1, 8, 128)
        assert torch.equal(out[0, 0, 0, 1], x[0, 0, 37])
        _same(out, _oracle(x, 1, 64, 8), f"needle {dtype}")
    x = torch.randn(1, 1, 67, 4)
    last = _proto_pool_seq(x.to(DEV), 64, 8)[0, 0, 1].cpu()
    torch.testing.assert_close(last[0], x[0, 0, 64:].mean(dim=0), atol=1e-5, rtol=0)
    assert not (last == 0).all(dim=-1).any()


@pytest.mark.parametrize("dtype,B,H,G,L,d,block,P,layout", [
    (torch.bfloat16, 1, 28, 4, 1000, 128, 64, 8, "bthd"),
    (torch.bfloat16, 2, 4, 4, 700, 128, 64, 8, "bhtd"),
    (torch.float16, 1, 8, 2, 333, 64, 64, 8, "bthd"),
    (torch.float32, 1, 6, 3, 260, 32, 64, 8, "bhtd"),
    (torch.bfloat16, 1, 4, 2, 150, 4, 64, 8, "bhtd"),     # head_dim 4: scalar path
    (torch.float16, 1, 2, 1, 100, 16, 8, 12, "bhtd"),     # block 8, P > block + 1
    (torch.bfloat16, 1, 16, 2, 190, 128, 64, 8, "bhtd"),  # 8 heads per group, ragged last block
    (torch.float16, 2, 6, 2, 129, 96, 64, 8, "bthd"),     # 3 heads per group, 12 chunks per token
    (torch.float16, 1, 4, 4, 333, 128, 64, 8, "bthd"),    # one head per group (16-bit tile), strided rows, ragged block
    (torch.bfloat16, 1, 3, 3, 200, 64, 32, 8, "bhtd"),    # one head per group, 32-token blocks, ragged block
])
def test_proto_pool_matches_oracle(dtype, B, H, G, L, d, block, P, layout):
    g = torch.Generator().manual_seed(L + H)
    if layout == "bthd":
        x = torch.randn(B, L, H, d, generator=g).to(dtype).transpose(1, 2)
    else:
        x = torch.randn(B, H, L, d, generator=g).to(dtype)
    x[:, :, 5] *= 30.0                                   # planted outlier rows
    xd = x.to(DEV) if layout == "bhtd" else x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    got = proto_pool_grouped(xd, G, block, P)
    _same(got, _oracle(x, G, block, P), "grouped")
    if G != H:
        avg = _group_avg_tokens(xd, G)
        _same(avg, osel.group_avg(x.float().numpy(), G, _NAMES[dtype]), "group avg")
        _same(_proto_pool_seq(avg, block, P), _oracle(x, G, block, P), "two-step")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_key_side_keeps_negative_zero(dtype):
    # One head per group: tokens enter the tile unchanged (no averaging), so
    # an outlier row holding -0.0 is emitted with its sign bits (value
    # equality alone would not see a -0 -> +0 change).
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 2, 128, 64, generator=g).to(dtype)
    x[:, :, 9] = 40.0
    x[:, :, 9, ::3] = -0.0
    got = _proto_pool_seq(x.to(DEV), 64, 8).float().cpu().numpy()
    exp = _oracle(x, 2, 64, 8)
    _same(torch.from_numpy(got), exp, "values")
    assert np.array_equal(np.signbit(got), np.signbit(exp))
    assert np.signbit(got[0, :, 0, 1, ::3]).all()      # the planted row is prototype 1 of block 0


def test_full_size_cfg3_one_group_and_invariants():
    print("cfg3 protos: generating inputs", flush=True)
    q, k, _ = workloads.qkv(0, 65536, 28, 4, 128, torch.bfloat16, use_rope=False, layout="bthd")
    qd = q.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    kd = k.to(DEV)
    pq = proto_pool_grouped(qd, 4)
    pk = _proto_pool_seq(kd, 64, 8)
    torch.cuda.synchronize()
    assert pq.shape == (1, 4, 1024, 8, 128) and pk.shape == (1, 4, 1024, 8, 128)
    print("cfg3 protos: oracle for KV group 2", flush=True)
    _same(pq[:, 2:3], _oracle(q[:, 14:21], 1, 64, 8), "cfg3 q group 2")
    _same(pk[:, 2:3], _oracle(k[:, 2:3], 1, 64, 8), "cfg3 k group 2")
    # Mean prototype of every group equals the block mean of the group-averaged tokens.
    qm = q.float().reshape(1, 4, 7, 1024, 64, 128).mean(dim=(2, 4)).to(DEV)
    torch.testing.assert_close(pq[:, :, :, 0].float(), qm, atol=2e-2, rtol=1e-2)


# Query and key prototypes in one launch against the two launches, bit for
# bit: query heads per KV head 1, 4, 7 and 8, ragged L, blocks of 64 and 32,
# 8 and 3 prototypes, both 16-bit dtypes, [B, T, H, D] and [B, H, T, D]
# storage, head_dim 128 and 64.
@pytest.mark.parametrize("dtype,B,Hq,Hkv,L,d,block,P,bthd", [
    (torch.bfloat16, 1, 28, 4, 4097, 128, 64, 8, True),
    (torch.float16, 2, 8, 2, 1000, 128, 64, 8, False),
    (torch.bfloat16, 1, 8, 1, 130, 64, 32, 3, True),
    (torch.float16, 1, 4, 4, 777, 128, 64, 8, True),
    (torch.bfloat16, 2, 16, 2, 65, 128, 64, 65, False),
])
def test_proto_pool_qk_equals_two_launches(dtype, B, Hq, Hkv, L, d, block, P, bthd):
    from teacher.chunked_extract import _proto_pool_seq, proto_pool_grouped, proto_pool_qk
    print(f"proto_pool_qk {dtype} B={B} Hq={Hq} Hkv={Hkv} L={L} d={d} block={block} P={P}", flush=True)
    g = torch.Generator().manual_seed(L + Hq)
    if bthd:
        q = torch.randn(B, L, Hq, d, generator=g).to(dtype).to("cuda").transpose(1, 2)
        k = torch.randn(B, L, Hkv, d, generator=g).to(dtype).to("cuda").transpose(1, 2)
    else:
        q = torch.randn(B, Hq, L, d, generator=g).to(dtype).to("cuda")
        k = torch.randn(B, Hkv, L, d, generator=g).to(dtype).to("cuda")
    k[0, 0, 3, :8] = -0.0   # negative zeros survive the key side
    fq, fk = proto_pool_qk(q, k, block, P)
    eq, ek = proto_pool_grouped(q, Hkv, block, P), _proto_pool_seq(k, block, P)
    torch.cuda.synchronize()
    assert torch.equal(fq.view(torch.int16), eq.view(torch.int16))
    assert torch.equal(fk.view(torch.int16), ek.view(torch.int16))
