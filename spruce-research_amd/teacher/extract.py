"""Eager attention maps from a Hugging Face model (teacher/extract.py:3-14)."""
import torch


def get_attentions(model, tok, prompt, device="cuda"):
    """Per-layer [batch, heads, seq, seq] attention probabilities and the prompt length."""
    inputs = tok(prompt, return_tensors="pt").to(device)
    with torch.no_grad():
        outputs = model(**inputs, output_attentions=True)
    attentions = outputs.attentions
    if not (isinstance(attentions, tuple) and len(attentions) > 0):
        raise AssertionError("Attentions not returned by the model.")
    if attentions[0].dim() != 4:
        raise AssertionError(
            f"Unexpected attention tensor shape. got shape {tuple(attentions[0].shape)}, expected 4D tensor.")
    return attentions, inputs["input_ids"].shape[1]
