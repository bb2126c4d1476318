"""Top-down key-tree traversal, under the reference's module name.

``traverse_to_leaf_ids``, ``traverse_to_leaf``, ``leaf_ids_to_mask`` and
``child_parent_index`` are this build's (``selector.traversal``: one HIP
launch walks every query row; reference scripts/eval_tree_traversal.py:42-142).
``load_gate`` (reference :26-32) restores a ``FlatGate`` checkpoint with a
weights-only load.  The evaluation helpers and the command-line driver
(``expand_paths``, ``leaf_metrics``, ``format_budget_metrics``, ``main``) are
the checkout's own, reached through the module ``__getattr__``;
``python -m scripts.eval_tree_traversal`` runs that driver with this module's
functions.
"""
import torch

from selector.gate import FlatGate
from selector.traversal import (child_parent_index, leaf_ids_to_mask, traverse_to_leaf,
                                traverse_to_leaf_ids)
from spruce_hip.overlay import forward_missing, run_upstream_main

__all__ = ["child_parent_index", "leaf_ids_to_mask", "load_gate", "traverse_to_leaf",
           "traverse_to_leaf_ids"]


def load_gate(path, device):
    """``(gate, config)`` from a checkpoint holding ``config`` (num_layers,
    head_dim, proj_dim) and the gate's ``state_dict``; the gate is in eval mode
    on ``device``.  The file is read with ``weights_only=True``: tensors and
    plain containers only, nothing in it is executed."""
    ckpt = torch.load(path, map_location=device, weights_only=True)
    cfg = ckpt["config"]
    gate = FlatGate(cfg["num_layers"], cfg["head_dim"], cfg["proj_dim"]).to(device)
    gate.load_state_dict(ckpt["state_dict"])
    gate.eval()
    return gate, cfg


__getattr__ = forward_missing("scripts.eval_tree_traversal", __file__)

if __name__ == "__main__":
    import sys

    sys.exit(run_upstream_main("scripts.eval_tree_traversal", __file__, {
        "load_gate": load_gate,
        "child_parent_index": child_parent_index,
        "traverse_to_leaf_ids": traverse_to_leaf_ids,
        "traverse_to_leaf": traverse_to_leaf,
        "leaf_ids_to_mask": leaf_ids_to_mask,
    }))
