"""Script modules of the reference whose library functions this build replaces.

``scripts.export_selected_blocks`` (route packing) and
``scripts.eval_tree_traversal`` (gate loading and the top-down key-tree walk)
are imported by the reference's live-route benchmarks; here they resolve to the
HIP implementations.  Every other ``scripts.*`` module, and the names these
two do not define, come from a reference checkout further down ``sys.path``.
"""
from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)
