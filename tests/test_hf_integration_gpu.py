"""Hugging Face integration on the GPU with a small random-init Qwen2 model.

No checkpoint is available offline, so the model is Qwen2 architecture with
random weights (2 layers, 7 query heads over 1 KV head, head_dim 64).

* All-causal-blocks equivalence (the reference's acceptance check,
  benchmarks/all_blocks_equivalence.py:44-50,159-174 there): the registered
  HIP sparse-prefill attention with every causal block selected gives the
  same last hidden state as torch's dense causal SDPA.  Bar: 2e-2 max-abs and
  1e-3 mean-abs after normalising by the hidden state's RMS.
* Prefill then decode: the cached one-token step goes to SDPA (decode stays
  dense, kernels/sparse_prefill.py:63-66 there); last-token and decoded
  logits within 2e-2 of the logits RMS of a bf16-input SDPA run, same token.
* Teacher capture (get_pooled_targets, teacher/chunked_extract.py:216-265
  there): per-layer pooled mass equals pool_attention of the model's eager
  attention maps (the reference's integration check,
  tests/validate_chunked_extract.py:24-54), within 2e-2 max-abs /
  1e-3 mean-abs of mass divided by the 64 rows of a block; prototypes have
  the reference's shapes and dtype.
The model runs in float32 (the kernels round Q/K/V to bfloat16 for the
matrix cores), which keeps torch's eager bf16 batched products out of the test.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _model():
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(vocab_size=256, hidden_size=448, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=7, num_key_value_heads=1, max_position_embeddings=2048,
                      rope_theta=1e6, attn_implementation="sdpa")
    torch.manual_seed(0)
    return Qwen2ForCausalLM(cfg).to(DEV).eval()


def _set_impl(model, name):
    model.config._attn_implementation = name
    for m in model.modules():
        c = getattr(m, "config", None)
        if c is not None:
            c._attn_implementation = name


def _bf16_input_sdpa(module, query, key, value, attention_mask, **kwargs):
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    r = lambda t: t.to(torch.bfloat16).to(t.dtype)
    kwargs.pop("selected_blocks", None)
    kwargs.pop("block_size", None)
    return sdpa_attention_forward(module, r(query), r(key), r(value), attention_mask, **kwargs)


@torch.no_grad()
def test_all_causal_blocks_match_dense_sdpa():
    from transformers import AttentionInterface
    from kernels.sparse_prefill import register_triton_sparse_prefill_attention
    model = _model()
    T = 300
    ids = torch.randint(0, 256, (1, T), generator=torch.Generator().manual_seed(1)).to(DEV)
    AttentionInterface.register("bf16_input_sdpa", _bf16_input_sdpa)
    _set_impl(model, "bf16_input_sdpa")
    dense = model.model(input_ids=ids, use_cache=False).last_hidden_state
    qb = (T + 63) // 64
    sel = torch.full((1, 2, 1, qb, qb), -1, dtype=torch.int32)
    for q in range(qb):
        sel[0, :, 0, q, : q + 1] = torch.arange(q + 1, dtype=torch.int32)
    name = register_triton_sparse_prefill_attention()
    _set_impl(model, name)
    sparse = model.model(input_ids=ids, use_cache=False, selected_blocks=sel.to(DEV), block_size=64).last_hidden_state
    rms = dense.pow(2).mean().sqrt()
    d = ((sparse - dense).abs() / rms)
    print(f"all-blocks hidden: max_abs={d.max().item():.3e} mean_abs={d.mean().item():.3e}", flush=True)
    assert d.max().item() <= 2e-2 and d.mean().item() <= 1e-3


@torch.no_grad()
def test_get_pooled_targets_matches_eager_attention_maps():
    from transformers import BatchEncoding
    from teacher.chunked_extract import get_pooled_targets
    from teacher.extract import get_attentions
    from teacher.pool import pool_attention
    from teacher.validate import check_causal

    class Tok:
        def __call__(self, prompt, return_tensors="pt"):
            return BatchEncoding({"input_ids": torch.tensor([prompt])})

    model = _model()
    prompt = torch.randint(0, 256, (200,), generator=torch.Generator().manual_seed(2)).tolist()
    pooled, pq, pk, seq_len = get_pooled_targets(model, Tok(), prompt, device=DEV)
    assert seq_len == 200 and pooled.shape == (1, 2, 7, 4, 4) and pooled.device.type == "cpu"
    assert pq.shape == (1, 2, 1, 4, 8, 64) and pk.shape == (1, 2, 1, 4, 8, 64) and pq.dtype == torch.float32
    _set_impl(model, "eager")
    attns, n = get_attentions(model, Tok(), prompt, device=DEV)
    for layer in range(2):
        ref = pool_attention(attns[layer].float(), 64).cpu()
        assert check_causal(pooled[:, layer]) == (True, None)
        d = (pooled[:, layer] - ref).abs() / 64
        print(f"layer {layer} mass: max_abs={d.max().item():.3e} mean_abs={d.mean().item():.3e}", flush=True)
        assert d.max().item() <= 2e-2 and d.mean().item() <= 1e-3


@torch.no_grad()
def test_prefill_then_decode_dispatches_decode_to_sdpa():
    # SPRUCE keeps decode dense (kernels/sparse_prefill.py:63-66 in the
    # reference): the cached one-token step goes to SDPA with its mask while
    # selected_blocks keeps being forwarded.  Logits of the prefill's last
    # token and of the decoded token match a bf16-input SDPA run.
    model = _model()
    T = 200
    ids = torch.randint(0, 256, (1, T), generator=torch.Generator().manual_seed(3)).to(DEV)
    qb = (T + 63) // 64
    sel = torch.full((1, 2, 1, qb, qb), -1, dtype=torch.int32)
    for q in range(qb):
        sel[0, :, 0, q, : q + 1] = torch.arange(q + 1, dtype=torch.int32)
    sel = sel.to(DEV)

    def run(name):
        _set_impl(model, name)
        out = model(input_ids=ids, use_cache=True, selected_blocks=sel, block_size=64)
        nxt = out.logits[:, -1:].argmax(-1)
        step = model(input_ids=nxt, past_key_values=out.past_key_values, use_cache=True,
                     selected_blocks=sel, block_size=64)
        return out.logits[:, -1], step.logits[:, -1], nxt

    from transformers import AttentionInterface
    from kernels.sparse_prefill import register_triton_sparse_prefill_attention
    AttentionInterface.register("bf16_input_sdpa", _bf16_input_sdpa)
    dense_last, dense_step, dense_next = run("bf16_input_sdpa")
    sparse_last, sparse_step, sparse_next = run(register_triton_sparse_prefill_attention())
    for a, b in ((sparse_last, dense_last), (sparse_step, dense_step)):
        rms = b.pow(2).mean().sqrt()
        d = ((a - b).abs() / rms).max().item()
        print(f"logits max_abs/rms={d:.3e}", flush=True)
        assert d <= 2e-2
    assert torch.equal(sparse_next, dense_next)
