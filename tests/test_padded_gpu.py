"""Padded-batch prefill through the HIP kernels (sparse/attention.py:147-150,
173-176, 225-229 in the reference): a 4-D decoder mask reduced to key
validity, applied inside the direct-index kernel, and excluded from the
residual summary table.

Bar: 2e-2 max-abs / 1e-3 mean-abs against the float32 oracle at the real
query positions (outputs at padding positions are not defined).  Batch row 0
is right-padded, row 1 left-padded.
"""
import numpy as np
import pytest
import torch

import oracle.attention as ora
import oracle.summaries as osum
from interfaces.residual_summaries import build_residual_summary_nodes
from kernels.direct_index import direct_index_sparse_prefill
from sparse.attention import sparse_prefill_attention_forward

pytestmark = pytest.mark.gpu
DEV = "cuda"
MAX_ABS, MEAN_ABS = 2e-2, 1e-3


class _Module(torch.nn.Module):
    layer_idx = 0


def _case(seed, Hq, Hkv, T, D, dtype, right_len, left_pad, extra=3):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(2, T, Hq, D, generator=gen).to(dtype).transpose(1, 2)
    k = torch.randn(2, T, Hkv, D, generator=gen).to(dtype).transpose(1, 2)
    v = torch.randn(2, T, Hkv, D, generator=gen).to(dtype).transpose(1, 2)
    valid = torch.zeros(2, T, dtype=torch.bool)
    valid[0, :right_len] = True
    valid[1, left_pad:] = True
    causal = torch.tril(torch.ones(T, T, dtype=torch.bool))
    mask = (causal[None] & valid[:, None, :])[:, None]            # sdpa_mask layout
    Q = (T + 63) // 64
    rng = np.random.default_rng(seed)
    sel = np.full((2, 1, Hkv, Q, extra + 2), -1, np.int32)
    for b, g, qb in np.ndindex(2, Hkv, Q):
        pick = rng.choice(qb + 1, size=min(qb + 1, extra), replace=False).tolist()
        row = sorted(set(pick) | {qb, max(0, qb - 1)})
        sel[b, 0, g, qb, : len(row)] = row
    return q, k, v, valid, mask, torch.from_numpy(sel)


def _dev(*xs):
    return [x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in xs]


def _check_real_rows(out, expected, valid, what):
    a = out.float().cpu().numpy().astype(np.float64)
    rows = valid.numpy()
    d = np.abs(a - expected)[rows]
    print(f"{what}: max_abs={d.max():.3e} mean_abs={d.mean():.3e}", flush=True)
    assert np.isfinite(a[rows]).all()
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, (what, d.max(), d.mean())


@pytest.mark.parametrize("Hq,Hkv,T,D,dtype", [
    (28, 4, 700, 128, torch.bfloat16),   # Qwen2-7B heads, producer-wave form
    (8, 2, 333, 64, torch.float16),      # G=4, full 8-wave parts
    (6, 2, 260, 128, torch.float32),
])
def test_padded_batch_matches_oracle(Hq, Hkv, T, D, dtype):
    q, k, v, valid, mask, sel = _case(T + Hq, Hq, Hkv, T, D, dtype, right_len=T - 210, left_pad=130)
    qd, kd, vd = _dev(q, k, v)
    out, _ = sparse_prefill_attention_forward(
        _Module(), qd, kd, vd, mask.to(DEV), selected_blocks=sel.to(DEV), block_size=64,
        validate_selected_blocks_input=False)
    torch.cuda.synchronize()
    expected = ora.sparse_attention_index(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                          sel[:, 0].numpy(), key_valid=valid.numpy())
    _check_real_rows(out, expected, valid, f"padded Hq{Hq} Hkv{Hkv} T{T} D{D} {dtype}")
    direct = direct_index_sparse_prefill(qd, kd, vd, sel[:, 0].contiguous().to(DEV), scale=D ** -0.5,
                                         key_valid=valid.to(DEV))
    assert torch.equal(direct, out)
    # Left padding changes real rows (the padding keys would otherwise count).
    plain = direct_index_sparse_prefill(qd, kd, vd, sel[:, 0].contiguous().to(DEV), scale=D ** -0.5)
    assert (plain[1, 130:].float() - out[1, 130:].float()).abs().max().item() > 1e-2


def test_all_real_tokens_mask_equals_unmasked():
    q, k, v, _, _, sel = _case(5, 28, 4, 512, 128, torch.bfloat16, right_len=512, left_pad=0)
    qd, kd, vd = _dev(q, k, v)
    ones = torch.tril(torch.ones(512, 512, dtype=torch.bool))[None, None].expand(2, 1, 512, 512).contiguous()
    with_mask, _ = sparse_prefill_attention_forward(
        _Module(), qd, kd, vd, ones.to(DEV), selected_blocks=sel.to(DEV), block_size=64,
        validate_selected_blocks_input=False)
    without, _ = sparse_prefill_attention_forward(
        _Module(), qd, kd, vd, None, selected_blocks=sel.to(DEV), block_size=64,
        validate_selected_blocks_input=False)
    forced = direct_index_sparse_prefill(qd, kd, vd, sel[:, 0].contiguous().to(DEV), scale=128 ** -0.5,
                                         key_valid=torch.ones(2, 512, dtype=torch.bool, device=DEV))
    torch.cuda.synchronize()
    assert torch.equal(with_mask, without) and torch.equal(forced, without)


@pytest.mark.parametrize("P", [1, 4])
def test_padded_batch_with_residual_summaries(P):
    q, k, v, valid, mask, sel = _case(31 + P, 28, 4, 640, 128, torch.bfloat16, right_len=400, left_pad=150)
    qd, kd, vd = _dev(q, k, v)
    residual = build_residual_summary_nodes(sel.to(DEV))
    out, _ = sparse_prefill_attention_forward(
        _Module(), qd, kd, vd, mask.to(DEV), selected_blocks=sel.to(DEV), block_size=64,
        validate_selected_blocks_input=False, residual_summaries=True, residual_summary_nodes=residual,
        summary_prototypes=P)
    torch.cuda.synchronize()
    kn, vn = k.float().numpy(), v.float().numpy()
    Q = sel.shape[3]
    lay = osum.tree_layout(Q)
    rs, re = osum.token_ranges(lay["starts"], lay["ends"], kn.shape[2], 64, P)
    keys, vals, _, logc = osum.kv_summary(kn, vn, rs, re, valid.numpy())
    N = len(lay["starts"])
    expected = ora.sparse_attention_summaries(
        q.float().numpy(), kn, vn, sel[:, 0].numpy(), residual[:, 0].cpu().numpy(),
        keys.reshape(2, 4, N, P, 128), vals.reshape(2, 4, N, P, 128), logc.reshape(2, N, P),
        key_valid=valid.numpy())
    _check_real_rows(out, expected, valid, f"padded summaries P{P}")


@torch.no_grad()
def test_padded_batch_through_a_qwen2_model():
    # A right- and a left-padded prompt through the registered HIP backend
    # (every causal block selected) against Transformers' SDPA with the same
    # padding mask, in float32 weights; hidden states compared at real tokens.
    from transformers import AttentionInterface, Qwen2Config, Qwen2ForCausalLM
    from sparse.attention import register_sparse_prefill_attention
    cfg = Qwen2Config(vocab_size=256, hidden_size=448, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=7, num_key_value_heads=1, max_position_embeddings=2048,
                      rope_theta=1e6, attn_implementation="sdpa")
    torch.manual_seed(0)
    model = Qwen2ForCausalLM(cfg).to(DEV).eval()
    T = 300
    ids = torch.randint(0, 256, (2, T), generator=torch.Generator().manual_seed(4)).to(DEV)
    am = torch.ones(2, T, dtype=torch.long, device=DEV)
    am[0, 220:] = 0
    am[1, :90] = 0

    def bf16_inputs_sdpa(module, query, key, value, attention_mask, **kwargs):
        from transformers.integrations.sdpa_attention import sdpa_attention_forward
        for name in ("selected_blocks", "block_size", "validate_selected_blocks_input"):
            kwargs.pop(name, None)
        r = lambda t: t.to(torch.bfloat16).to(t.dtype)  # noqa: E731
        return sdpa_attention_forward(module, r(query), r(key), r(value), attention_mask, **kwargs)

    def set_impl(name):
        model.config._attn_implementation = name
        for m in model.modules():
            c = getattr(m, "config", None)
            if c is not None:
                c._attn_implementation = name

    from transformers import AttentionMaskInterface
    from transformers.masking_utils import sdpa_mask
    AttentionInterface.register("bf16_inputs_sdpa_padded", bf16_inputs_sdpa)
    AttentionMaskInterface.register("bf16_inputs_sdpa_padded", sdpa_mask)
    set_impl("bf16_inputs_sdpa_padded")
    dense = model.model(input_ids=ids, attention_mask=am, use_cache=False).last_hidden_state
    qb = (T + 63) // 64
    sel = torch.full((2, 2, 1, qb, qb), -1, dtype=torch.int32)
    for q in range(qb):
        sel[:, :, 0, q, : q + 1] = torch.arange(q + 1, dtype=torch.int32)
    set_impl(register_sparse_prefill_attention())
    sparse = model.model(input_ids=ids, attention_mask=am, use_cache=False, selected_blocks=sel.to(DEV),
                         block_size=64).last_hidden_state
    real = am.bool()
    rms = dense[real].pow(2).mean().sqrt()
    d = (sparse[real] - dense[real]).abs() / rms
    print(f"padded batch hidden: max_abs/rms={d.max().item():.3e} mean_abs/rms={d.mean().item():.3e}",
          flush=True)
    assert torch.isfinite(sparse[real]).all()
    assert d.max().item() <= 2e-2 and d.mean().item() <= 1e-3
