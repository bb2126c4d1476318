"""Route packing into the selected_blocks contract, under the reference's module name.

``selected_mask_to_blocks`` and ``selected_ids_to_blocks`` are the HIP route
packers of ``interfaces.packing`` (reference scripts/export_selected_blocks.py:38-175:
same arguments, policy and errors).  The file-handling helpers and the
command-line driver (``expand_paths``, ``safe_stem``, ``main``,
reference :26-36, :178-246) are the checkout's own, reached through the
module ``__getattr__``; ``python -m scripts.export_selected_blocks`` runs that
driver with the packers and the traversal of this package.
"""
from interfaces.packing import selected_ids_to_blocks, selected_mask_to_blocks
from interfaces.validator import PAD_VALUE
from scripts.eval_tree_traversal import load_gate, traverse_to_leaf_ids
from spruce_hip.overlay import forward_missing, run_upstream_main

__all__ = ["PAD_VALUE", "selected_ids_to_blocks", "selected_mask_to_blocks"]

__getattr__ = forward_missing("scripts.export_selected_blocks", __file__)

if __name__ == "__main__":
    run_upstream_main("scripts.export_selected_blocks", __file__, {
        "selected_ids_to_blocks": selected_ids_to_blocks,
        "selected_mask_to_blocks": selected_mask_to_blocks,
        "load_gate": load_gate,
        "traverse_to_leaf_ids": traverse_to_leaf_ids,
    })
