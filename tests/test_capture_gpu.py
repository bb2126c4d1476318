"""Dense causal prefill with selector-feature capture on the GPU
(``spruce_causal_prefill`` through the C ABI, and the capture hooks that use it).

Bars:
  * attention output: bit for bit the direct-index kernel run over the full
    ascending causal list (the same per-wave arithmetic; that kernel is pinned
    to the oracle in test_attention_gpu.py), and within 2e-2 (bf16) / 4e-3
    (f16) max-abs of the float64 dense causal oracle;
  * group-averaged queries, key prototypes and pooled query prototypes: bit for
    bit the standalone kernels (spruce_group_avg_tokens, spruce_proto_pool,
    proto_pool_grouped) and oracle/proto.c.
Cases: 1, 2, 3, 4, 5, 7 and 8 query heads per KV head (one and two parts per
row), head_dim 64 and 128, bf16 and f16, ragged sequence ends (T = 1, 97,
130, 333), a single block, [B,T,H,D] storage as the HF hook passes it, batch
2, the reference's needle known answer, and the full cfg2 layer (T = 32768,
28/4 heads) against the standalone kernels.
"""

import numpy as np
import pytest
import torch

import oracle.attention as oatt
import oracle.selector as osel
import spruce_hip
from kernels.direct_index import direct_index_sparse_prefill
from teacher.chunked_extract import (_capture_features, _CAPTURE_QK, _group_avg_tokens, _proto_pool_seq,
                                     causal_prefill_features, proto_pool_grouped)

pytestmark = pytest.mark.gpu
DEV = "cuda"
_NAMES = {torch.float16: "float16", torch.bfloat16: "bfloat16"}

def _qkv(seed, B, H, G, T, D, dtype, layout):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    if layout == "bthd":
        q = torch.randn(B, T, H, D, generator=gen, device=DEV).to(dtype).transpose(1, 2)
        k = torch.randn(B, T, G, D, generator=gen, device=DEV).to(dtype).transpose(1, 2)
        v = torch.randn(B, T, G, D, generator=gen, device=DEV).to(dtype).transpose(1, 2)
    else:
        q = torch.randn(B, H, T, D, generator=gen, device=DEV).to(dtype)
        k = torch.randn(B, G, T, D, generator=gen, device=DEV).to(dtype)
        v = torch.randn(B, G, T, D, generator=gen, device=DEV).to(dtype)
    return q, k, v

def _full_lists(B, G, T):
    qb = (T + 63) // 64
    idx = torch.full((B, G, qb, qb), -1, dtype=torch.int32)
    for i in range(qb):
        idx[:, :, i, : i + 1] = torch.arange(i + 1, dtype=torch.int32)
    return idx.to(DEV)

def _raw_capture(q, k, v, scale, P):
    """One spruce_causal_prefill call; returns (out [B,T,H,D], q_grouped, k_protos)."""
    B, H, T, D = q.shape
    G = k.shape[1]
    out = torch.empty((B, T, H, D), device=DEV, dtype=q.dtype)
    qg = torch.empty((B, G, T, D), device=DEV, dtype=q.dtype)
    kp = torch.empty((B, G, (T + 63) // 64, P, D), device=DEV, dtype=q.dtype)
    rc = spruce_hip.lib().spruce_causal_prefill(
        spruce_hip.ptr(q), spruce_hip.strides(q), spruce_hip.ptr(k), spruce_hip.strides(k),
        spruce_hip.ptr(v), spruce_hip.strides(v), B, H, G, T, D, float(scale), spruce_hip.dtype_code(q),
        spruce_hip.ptr(out), spruce_hip.strides(out, order=(0, 2, 1, 3)), spruce_hip.ptr(qg), spruce_hip.ptr(kp),
        P, spruce_hip.stream_of(q))
    spruce_hip.check(rc, "spruce_causal_prefill")
    return out, qg, kp

def _same(got, want, what):
    g = got.float().cpu().numpy() if isinstance(got, torch.Tensor) else got
    w = want.float().cpu().numpy() if isinstance(want, torch.Tensor) else want
    assert g.shape == w.shape, (what, g.shape, w.shape)
    bad = np.argwhere(~((g == w) | (np.isnan(g) & np.isnan(w))))
    assert bad.size == 0, (what, bad[:5].tolist(), g[tuple(bad[0])], w[tuple(bad[0])])

@pytest.mark.parametrize("dtype,B,H,G,T,D,layout", [
    (torch.bfloat16, 1, 28, 4, 333, 128, "bthd"),   # Qwen2-7B heads: 7 per KV head, two parts
    (torch.float16, 2, 8, 2, 200, 64, "bhtd"),      # 4 per KV head: one part, both halves
    (torch.bfloat16, 1, 5, 1, 130, 128, "bthd"),    # 5 per KV head
    (torch.bfloat16, 1, 16, 2, 64, 128, "bhtd"),    # 8 per KV head, a single block
    (torch.float16, 1, 2, 2, 97, 128, "bhtd"),      # 1 per KV head: the copy path
    (torch.bfloat16, 1, 6, 2, 1, 64, "bthd"),       # 3 per KV head, one token
])
def test_capture_matches_standalone_kernels_and_oracle(dtype, B, H, G, T, D, layout):
    q, k, v = _qkv(T + H, B, H, G, T, D, dtype, layout)
    scale = D ** -0.5
    P = 8
    print(f"capture case dtype={dtype} B={B} H={H} G={G} T={T} D={D} layout={layout}", flush=True)
    out, qg, kp = _raw_capture(q, k, v, scale, P)
    torch.cuda.synchronize()
    # Attention: the direct-index kernel over every causal block, same order.
    ref = direct_index_sparse_prefill(q, k, v, _full_lists(B, G, T), scale, kernel_variant="tiled_gqa")
    _same(out, ref, "attention vs full-list direct index")
    want = oatt.dense_causal_attention(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                       v.float().cpu().numpy(), scale)
    tol = 2e-2 if dtype == torch.bfloat16 else 4e-3
    assert np.abs(out.float().cpu().numpy() - want).max() <= tol
    # Features: the standalone kernels and the oracle, bit for bit.
    _same(qg, _group_avg_tokens(q, G), "q_grouped vs spruce_group_avg_tokens")
    _same(kp, _proto_pool_seq(k, 64, P), "k_protos vs spruce_proto_pool")
    name = _NAMES[dtype]
    qa = q.float().cpu().numpy()
    qa_grouped = osel.group_avg(qa, G, name) if G != H else qa
    _same(qg, qa_grouped, "q_grouped vs oracle")
    _same(kp, osel.proto_pool(k.float().cpu().numpy(), 64, P, name), "k_protos vs oracle")
    # The host form pools the grouped queries: proto_pool_grouped(q) exactly.
    out2, pq, pk = causal_prefill_features(q, k, v, scale, P)
    _same(out2, out, "host form attention")
    _same(pk, kp, "host form key prototypes")
    _same(pq, proto_pool_grouped(q, G, 64, P), "pooled queries vs proto_pool_grouped")
    _same(pq, osel.proto_pool(qa_grouped, 64, P, name), "pooled queries vs oracle")

def test_capture_off_and_prototype_counts():
    q, k, v = _qkv(3, 1, 14, 2, 150, 128, torch.bfloat16, "bthd")
    scale = 0.1
    out, _, _ = causal_prefill_features(q, k, v, scale, capture=False)
    out_c, pq, pk = causal_prefill_features(q, k, v, scale, 8)
    _same(out, out_c, "capture on/off attention")
    for P in (1, 2, 65):
        _, pq2, pk2 = causal_prefill_features(q, k, v, scale, P)
        _same(pk2, _proto_pool_seq(k, 64, P), f"k_protos P={P}")
        _same(pq2, proto_pool_grouped(q, 2, 64, P), f"pooled queries P={P}")

def test_needle_known_answer():
    # The reference's needle check (a token far from its block's mean is kept
    # as prototype 1), on the key side of the fused pass.
    q, k, v = _qkv(5, 1, 7, 1, 128, 128, torch.bfloat16, "bhtd")
    k = (k * 0.01).contiguous()
    k[0, 0, 37, :] = 40.0
    _, _, pk = causal_prefill_features(q, k, v, 128 ** -0.5)
    assert torch.equal(pk[0, 0, 0, 1], k[0, 0, 37])
    _same(pk, _proto_pool_seq(k, 64, 8), "needle k_protos")

def test_capture_argument_errors():
    q, k, v = _qkv(7, 1, 4, 1, 64, 64, torch.bfloat16, "bhtd")
    with pytest.raises(ValueError, match="model dtype"):
        causal_prefill_features(q.float(), k.float(), v.float(), 0.1)
    q16, k16, v16 = _qkv(7, 1, 16, 1, 64, 64, torch.bfloat16, "bhtd")
    with pytest.raises(ValueError, match="at most 8"):
        causal_prefill_features(q16, k16, v16, 0.1)
    with pytest.raises(ValueError, match="P must be"):
        causal_prefill_features(q, k, v, 0.1, P=0)
    # Only one of the two capture outputs: rejected by the library.
    B, H, T, D = q.shape
    out = torch.empty((B, T, H, D), device=DEV, dtype=q.dtype)
    qg = torch.empty((B, 1, T, D), device=DEV, dtype=q.dtype)
    rc = spruce_hip.lib().spruce_causal_prefill(
        spruce_hip.ptr(q), spruce_hip.strides(q), spruce_hip.ptr(k), spruce_hip.strides(k),
        spruce_hip.ptr(v), spruce_hip.strides(v), B, H, 1, T, D, 0.1, 0,
        spruce_hip.ptr(out), spruce_hip.strides(out, order=(0, 2, 1, 3)), spruce_hip.ptr(qg), None, 8,
        spruce_hip.stream_of(q))
    assert rc != 0 and "both" in spruce_hip.last_error()
    # f32 with capture outputs: rejected by the library too.
    qf, kf, vf = (t.float() for t in (q, k, v))
    outf = torch.empty((B, T, H, D), device=DEV, dtype=torch.float32)
    kp = torch.empty((B, 1, 1, 8, D), device=DEV, dtype=torch.float32)
    qgf = qg.float()
    rc = spruce_hip.lib().spruce_causal_prefill(
        spruce_hip.ptr(qf), spruce_hip.strides(qf), spruce_hip.ptr(kf), spruce_hip.strides(kf),
        spruce_hip.ptr(vf), spruce_hip.strides(vf), B, H, 1, T, D, 0.1, 2,
        spruce_hip.ptr(outf), spruce_hip.strides(outf, order=(0, 2, 1, 3)), spruce_hip.ptr(qgf),
        spruce_hip.ptr(kp), 8, spruce_hip.stream_of(q))
    assert rc != 0 and "model dtype" in spruce_hip.last_error()

class _Layer:
    layer_idx = 3

def test_feature_capture_hook_uses_the_fused_pass():
    # "selector_feature_capture" (teacher/chunked_extract.py:163-181 in the
    # reference): returns [b, L, H, d] attention and records the prototypes.
    q, k, v = _qkv(11, 1, 14, 2, 260, 128, torch.bfloat16, "bthd")
    _CAPTURE_QK.clear()
    out, none = _capture_features(_Layer(), q, k, v, None, scaling=None)
    assert none is None and out.shape == (1, 260, 14, 128) and out.is_contiguous()
    pq, pk = _CAPTURE_QK.pop(3)
    assert pq.device.type == "cpu" and pq.dtype == torch.bfloat16 and pq.shape == (1, 2, 5, 8, 128)
    _same(pq, proto_pool_grouped(q, 2, 64, 8), "hook pooled queries")
    _same(pk, _proto_pool_seq(k, 64, 8), "hook pooled keys")
    want = oatt.dense_causal_attention(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                       v.float().cpu().numpy(), 128 ** -0.5)
    assert np.abs(out.float().cpu().numpy() - want).max() <= 2e-2

def test_full_size_cfg2_layer_against_standalone_kernels():
    # T = 32768, 28 query heads over 4 KV heads (the cfg2 layer), dense causal.
    from spruce_hip import workloads
    T, H, G, D = 32768, 28, 4, 128
    q, k, v = workloads.qkv(0, T, H, G, D, torch.bfloat16, use_rope=True, layout="bthd", device="cuda")
    print("full-size capture T=32768", flush=True)
    out, qg, kp = _raw_capture(q, k, v, D ** -0.5, 8)
    torch.cuda.synchronize()
    _same(qg, _group_avg_tokens(q, G), "full-size q_grouped")
    _same(kp, _proto_pool_seq(k, 64, 8), "full-size k_protos")
    # Attention: bit for bit the direct-index kernel over every causal block.
    ref = direct_index_sparse_prefill(q, k, v, _full_lists(1, G, T), D ** -0.5, kernel_variant="tiled_gqa")
    assert torch.equal(out, ref)
    assert torch.isfinite(out.float()).all()
