"""All-causal-blocks equivalence gate for the sparse-prefill path.

Drop-in for the gate functions of the reference's
benchmarks/all_blocks_equivalence.py: with every causal block selected the
sparse backend has no pruning decision left, so a model run through it must
match the same model run through dense attention.  The acceptance criteria
are the reference's (DEFAULT_ACCEPTANCE, :44-50): finite outputs, the same
top-1 next token, top-10 overlap >= 0.9, logits cosine >= 0.999 and final
hidden relative RMSE <= 0.02, on the last position's logits
(:260-262: output embeddings applied to the last hidden row).

The reference loads a checkpoint by hub name and reads prompt manifests;
neither is available offline, so ``run_equivalence`` takes a loaded model and
token ids from the caller.  The reference's manifest and model-loading
driver (``main``, ``load_manifest``, ``select_matched_records``, ...) is reached
through the module ``__getattr__`` when its checkout is on ``sys.path``, and
``python -m benchmarks.all_blocks_equivalence`` runs that driver; its
attention calls resolve to this package's kernels.
"""
import math

import torch

from interfaces.validator import PAD_VALUE, validate_selected_blocks
from spruce_hip.overlay import forward_missing, run_upstream_main

__getattr__ = forward_missing("benchmarks.all_blocks_equivalence", __file__)

DEFAULT_ACCEPTANCE = {
    "require_finite": True,
    "require_same_top1": True,
    "minimum_top10_overlap": 0.9,
    "minimum_logits_cosine": 0.999,
    "maximum_final_hidden_relative_rmse": 0.02,
}


def all_causal_selected_blocks(*, num_layers, num_kv_groups, seq_len, block_size=64):
    """``[1, L, G, Qb, Qb]`` int32 rows listing every causal block 0..q, PAD
    after the diagonal (reference :53-68); validated against the contract."""
    if min(num_layers, num_kv_groups, seq_len, block_size) < 1:
        raise ValueError("layers, groups, sequence length, and block size must be positive")
    qb = math.ceil(seq_len / block_size)
    cols = torch.arange(qb, dtype=torch.int32)
    rows = torch.where(cols[None, :] <= cols[:, None], cols[None, :].expand(qb, qb),
                       torch.full((qb, qb), PAD_VALUE, dtype=torch.int32))
    selected = rows.expand(1, num_layers, num_kv_groups, qb, qb).clone()
    validate_selected_blocks(selected)
    return selected


def tensor_error(actual, expected):
    """max/mean abs error, RMSE and RMSE relative to the expected tensor's RMS
    (reference :116-137), accumulated in float32."""
    if actual.shape != expected.shape:
        raise ValueError(f"shape mismatch: {tuple(actual.shape)} vs {tuple(expected.shape)}")
    a, e = actual.float(), expected.float()
    diff = a - e
    rmse = float(diff.square().mean().sqrt().item())
    ref_rms = float(e.square().mean().sqrt().item())
    return {
        "actual_finite": bool(torch.isfinite(actual).all().item()),
        "expected_finite": bool(torch.isfinite(expected).all().item()),
        "max_abs": float(diff.abs().max().item()),
        "mean_abs": float(diff.abs().mean().item()),
        "rmse": rmse,
        "reference_rms": ref_rms,
        "relative_rmse": rmse / ref_rms if ref_rms else float("inf"),
    }


def logits_error(actual, expected, *, top_k=10):
    """tensor_error plus cosine similarity, top-1 agreement and top-k overlap
    of the flattened logits (reference :140-157)."""
    out = tensor_error(actual, expected)
    a, e = actual.float().flatten(), expected.float().flatten()
    a_top = torch.topk(a, k=top_k).indices.tolist()
    e_top = torch.topk(e, k=top_k).indices.tolist()
    out["cosine"] = float(torch.nn.functional.cosine_similarity(a[None], e[None]).item())
    out["top1_same"] = a_top[0] == e_top[0]
    out["actual_top_ids"] = [int(i) for i in a_top]
    out["expected_top_ids"] = [int(i) for i in e_top]
    out["top10_overlap"] = len(set(a_top) & set(e_top)) / top_k
    return out


def passes_acceptance(logits, final_hidden, criteria=DEFAULT_ACCEPTANCE):
    """The reference's acceptance rule (:160-174) over logits_error and
    tensor_error results."""
    finite = all((logits["actual_finite"], logits["expected_finite"],
                  final_hidden["actual_finite"], final_hidden["expected_finite"]))
    checks = (
        finite or not criteria["require_finite"],
        logits["top1_same"] or not criteria["require_same_top1"],
        logits["top10_overlap"] >= criteria["minimum_top10_overlap"],
        logits["cosine"] >= criteria["minimum_logits_cosine"],
        final_hidden["relative_rmse"] <= criteria["maximum_final_hidden_relative_rmse"],
    )
    return bool(all(checks))


def _set_backend(model, name):
    model.config._attn_implementation = name
    for module in model.modules():
        config = getattr(module, "config", None)
        if config is not None:
            config._attn_implementation = name


@torch.inference_mode()
def _run(model, input_ids, implementation, layer_outputs, **kwargs):
    _set_backend(model, implementation)
    handles = []
    for index, layer in enumerate(model.base_model.layers):
        def hook(_module, _inputs, output, index=index):
            hidden = output[0] if isinstance(output, (tuple, list)) else output
            layer_outputs.append((index, hidden.detach()))
        handles.append(layer.register_forward_hook(hook))
    try:
        output = model.base_model(input_ids=input_ids, use_cache=False, **kwargs)
    finally:
        for handle in handles:
            handle.remove()
    final_hidden = output.last_hidden_state.detach()
    logits = model.get_output_embeddings()(final_hidden[:, -1:, :])
    return final_hidden, logits.detach().float()


def run_equivalence(model, input_ids, *, dense_implementation, sparse_implementation, block_size=64,
                    kernel_variant=None, criteria=DEFAULT_ACCEPTANCE):
    """Runs ``model`` on ``input_ids`` (``[1, T]``) through the dense and the
    sparse attention backends (registered Transformers attention names), the
    sparse one with every causal block selected, and returns the logits and
    final-hidden errors, per-layer hidden errors and the acceptance verdict."""
    if input_ids.dim() != 2 or input_ids.shape[0] != 1:
        raise ValueError("input_ids must be [1, T]")
    config = model.config
    selected = all_causal_selected_blocks(
        num_layers=config.num_hidden_layers, num_kv_groups=config.num_key_value_heads,
        seq_len=input_ids.shape[1], block_size=block_size).to(input_ids.device)
    dense_layers, sparse_layers = [], []
    dense_hidden, dense_logits = _run(model, input_ids, dense_implementation, dense_layers)
    kwargs = dict(selected_blocks=selected, block_size=block_size, validate_selected_blocks_input=False)
    if kernel_variant is not None:
        kwargs["kernel_variant"] = kernel_variant
    sparse_hidden, sparse_logits = _run(model, input_ids, sparse_implementation, sparse_layers, **kwargs)
    logits = logits_error(sparse_logits, dense_logits)
    hidden = tensor_error(sparse_hidden, dense_hidden)
    layers = [{"layer": i, **tensor_error(s, d)} for (i, s), (_, d) in zip(sparse_layers, dense_layers)]
    return {"logits": logits, "final_hidden": hidden, "layers": layers,
            "accepted": passes_acceptance(logits, hidden, criteria)}


if __name__ == "__main__":
    run_upstream_main("benchmarks.all_blocks_equivalence", __file__, {})
