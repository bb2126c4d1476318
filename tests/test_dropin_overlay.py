"""The package as a drop-in in front of a reference checkout (CPU only).

A stand-in checkout is written into ``tmp_path``: the reference's package
names, with regular packages where the reference has an ``__init__.py``
(``sparse``, ``kernels``, ``benchmarks``) and namespace packages where it has
none (``selector``, ``teacher``, ``interfaces``, ``scripts``).  Its modules
are stubs written here: each records ``ORIGIN = "stand-in"``.  With
``spruce-research_amd/`` first on ``sys.path`` and the stand-in after it, a
subprocess imports the names the reference's callers import
(benchmarks/compare_dense_sparse_live_tree.py:27-79,
scripts/run_sparse_prefill_replay.py:22-44) and reports where each came from:
the hot-path modules must be this package's, every module this build does not
ship must be the checkout's, and names a partial module lacks must be
forwarded to the checkout's file of the same name.
"""
import argparse
import json
import os
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "spruce-research_amd")

STAND_IN = {
    # regular packages in the reference
    "sparse/__init__.py": "ORIGIN = 'stand-in'\n",
    "sparse/config.py": "ORIGIN = 'stand-in'\n",
    "sparse/attention.py": "ORIGIN = 'stand-in'\n",
    "sparse/plotting.py": "ORIGIN = 'stand-in'\ndef save_sparse_replay_plot(*a, **k):\n    return 'plot'\n",
    "kernels/__init__.py": "ORIGIN = 'stand-in'\n",
    "kernels/sparse_prefill.py": "ORIGIN = 'stand-in'\n",
    "benchmarks/__init__.py": "ORIGIN = 'stand-in'\n",
    "benchmarks/compare_dense_sparse.py":
        "ORIGIN = 'stand-in'\ndef _set_attention_backend(model, name):\n    return name\n",
    "benchmarks/all_blocks_equivalence.py": textwrap.dedent("""\
        ORIGIN = 'stand-in'
        def select_matched_records(records):
            return 'matched'
        def passes_acceptance(*a, **k):
            return 'stand-in'
        """),
    # namespace packages in the reference (no __init__.py)
    "selector/recall.py": "ORIGIN = 'stand-in'\n",
    "selector/loss.py": "ORIGIN = 'stand-in'\ndef kl_loss(*a):\n    return 0.0\n",
    "selector/tree.py": textwrap.dedent("""\
        ORIGIN = 'stand-in'
        from selector.loss import kl_loss
        def build_key_tree(*a, **k):
            return 'stand-in'
        def build_target_tree(*a, **k):
            return 'target tree'
        def iter_tree_levels(*a, **k):
            return build_key_tree()
        """),
    "teacher/prompt_replay.py":
        "ORIGIN = 'stand-in'\ndef reconstruct_teacher_prompt(*a):\n    return 'prompt'\n",
    "teacher/chunked_extract.py": "ORIGIN = 'stand-in'\n_HEAD_CHUNK = 2\n",
    "interfaces/validator.py": "ORIGIN = 'stand-in'\n",
    "scripts/route_overrides.py": "ORIGIN = 'stand-in'\ndef load_route_overrides(*a):\n    return {}\n",
    "scripts/export_selected_blocks.py": textwrap.dedent("""\
        ORIGIN = 'stand-in'
        def selected_ids_to_blocks(*a, **k):
            return 'stand-in'
        def expand_paths(patterns):
            return list(patterns)
        def main():
            # The command-line driver reports which packer it would call.
            print('packer=' + selected_ids_to_blocks.__module__)
        """),
    "scripts/eval_tree_traversal.py": textwrap.dedent("""\
        ORIGIN = 'stand-in'
        def traverse_to_leaf_ids(*a, **k):
            return 'stand-in'
        def leaf_metrics(*a, **k):
            return {'recall': 1.0}
        def main():
            print('traversal=' + traverse_to_leaf_ids.__module__)
            return 0
        """),
}

# Import statements of the reference's callers, one (module, names) pair each.
CALLER_IMPORTS = [
    ("interfaces.residual_summaries", ["build_residual_summary_nodes",
                                       "validate_residual_summary_nodes"]),
    ("interfaces.validator", ["validate_selected_blocks"]),
    ("kernels.sparse_prefill", ["SPRUCE_TRITON_SPARSE_PREFILL",
                                "register_triton_sparse_prefill_attention"]),
    ("scripts.eval_tree_traversal", ["load_gate", "traverse_to_leaf_ids"]),
    ("scripts.export_selected_blocks", ["selected_ids_to_blocks"]),
    ("scripts.route_overrides", ["load_route_overrides"]),
    ("selector.targets", ["load_selector_features", "load_teacher"]),
    ("selector.tree", ["build_key_tree"]),
    ("sparse.attention", ["SPARSE_PREFILL_ATTENTION", "register_sparse_prefill_attention",
                          "token_validity_from_attention_mask"]),
    ("sparse.config", ["ResidualSummaryConfig", "add_residual_summary_arguments",
                       "residual_summary_config_from_args"]),
    ("sparse.plotting", ["save_sparse_replay_plot"]),
    ("sparse.summaries", ["residual_attention_density"]),
    ("teacher.prompt_replay", ["reconstruct_teacher_prompt"]),
    ("benchmarks.compare_dense_sparse", ["_set_attention_backend"]),
]

PROBE = textwrap.dedent("""\
    import importlib, json, sys
    sys.path[:0] = [{pkg!r}, {stand_in!r}]
    calls = {calls!r}
    out = {{"modules": {{}}, "names": {{}}}}
    for module, names in calls:
        m = importlib.import_module(module)
        out["modules"][module] = m.__file__
        for name in names:
            value = getattr(m, name)
            out["names"][module + "." + name] = getattr(value, "__module__", module)
    import selector.tree, teacher.chunked_extract, benchmarks.all_blocks_equivalence, sparse
    out["forwarded"] = {{
        "selector.tree.build_target_tree": selector.tree.build_target_tree(),
        "selector.tree.iter_tree_levels": selector.tree.iter_tree_levels(),
        "teacher.chunked_extract._HEAD_CHUNK": teacher.chunked_extract._HEAD_CHUNK,
        "benchmarks.all_blocks_equivalence.select_matched_records":
            benchmarks.all_blocks_equivalence.select_matched_records([]),
        "scripts.eval_tree_traversal.leaf_metrics":
            importlib.import_module("scripts.eval_tree_traversal").leaf_metrics(),
        "sparse.save_sparse_replay_plot": sparse.save_sparse_replay_plot(),
    }}
    out["own"] = {{
        "benchmarks.all_blocks_equivalence.passes_acceptance":
            benchmarks.all_blocks_equivalence.passes_acceptance.__module__,
        "sparse.sparse_prefill_attention_forward": sparse.sparse_prefill_attention_forward.__module__,
    }}
    out["paths"] = {{p: list(importlib.import_module(p).__path__)
                    for p in ("sparse", "kernels", "benchmarks", "selector", "teacher",
                              "interfaces", "scripts")}}
    print(json.dumps(out))
    """)


def _write_stand_in(root):
    for rel, text in STAND_IN.items():
        path = root / rel
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(text)
    return root


def _run(code, cwd, args=()):
    env = dict(os.environ, PYTHONPATH="", PYTHONDONTWRITEBYTECODE="1")
    return subprocess.run([sys.executable, *args, "-c", code] if code else [sys.executable, *args],
                          cwd=cwd, env=env, capture_output=True, text=True, timeout=300)


def _is_ours(path):
    return os.path.realpath(path).startswith(os.path.realpath(PKG) + os.sep)


@pytest.fixture(scope="module")
def probe(tmp_path_factory):
    stand_in = _write_stand_in(tmp_path_factory.mktemp("checkout"))
    code = PROBE.format(pkg=PKG, stand_in=str(stand_in), calls=CALLER_IMPORTS)
    res = _run(code, cwd=str(stand_in.parent))
    assert res.returncode == 0, res.stderr[-3000:]
    return stand_in, json.loads(res.stdout.strip().splitlines()[-1])


def test_hot_path_modules_resolve_to_this_package(probe):
    _, out = probe
    for module in ("sparse.attention", "sparse.config", "sparse.summaries", "kernels.sparse_prefill",
                   "scripts.export_selected_blocks", "scripts.eval_tree_traversal", "selector.tree",
                   "selector.targets", "interfaces.validator", "interfaces.residual_summaries"):
        assert _is_ours(out["modules"][module]), (module, out["modules"][module])
    # The functions the live route calls are the HIP implementations.
    assert out["names"]["scripts.export_selected_blocks.selected_ids_to_blocks"] == "interfaces.packing"
    assert out["names"]["scripts.eval_tree_traversal.traverse_to_leaf_ids"] == "selector.traversal"
    assert out["names"]["scripts.eval_tree_traversal.load_gate"] == "scripts.eval_tree_traversal"
    assert out["names"]["selector.tree.build_key_tree"] == "selector.tree"
    assert out["own"]["sparse.sparse_prefill_attention_forward"] == "sparse.attention"
    assert out["own"]["benchmarks.all_blocks_equivalence.passes_acceptance"] == \
        "benchmarks.all_blocks_equivalence"


def test_modules_not_shipped_resolve_to_the_checkout(probe):
    stand_in, out = probe
    for module in ("sparse.plotting", "teacher.prompt_replay", "benchmarks.compare_dense_sparse",
                   "scripts.route_overrides"):
        path = out["modules"][module]
        assert os.path.realpath(path).startswith(os.path.realpath(str(stand_in))), (module, path)
    # Every package searches this build first, then the checkout.
    for package, path in out["paths"].items():
        assert _is_ours(path[0]) and any(
            os.path.realpath(p).startswith(os.path.realpath(str(stand_in))) for p in path[1:]), \
            (package, path)


def test_selector_recall_resolves_to_the_checkout(tmp_path):
    stand_in = _write_stand_in(tmp_path / "checkout")
    code = (f"import sys; sys.path[:0] = [{PKG!r}, {str(stand_in)!r}]\n"
            "import selector.recall as r; print(r.ORIGIN, r.__file__)")
    res = _run(code, cwd=str(tmp_path))
    assert res.returncode == 0, res.stderr[-2000:]
    origin, path = res.stdout.split()
    assert origin == "stand-in" and os.path.realpath(path).startswith(os.path.realpath(str(stand_in)))


def test_partial_modules_forward_missing_names(probe):
    _, out = probe
    assert out["forwarded"] == {
        "selector.tree.build_target_tree": "target tree",
        # The checkout's function runs in the checkout's module, with its own globals.
        "selector.tree.iter_tree_levels": "stand-in",
        "teacher.chunked_extract._HEAD_CHUNK": 2,
        "benchmarks.all_blocks_equivalence.select_matched_records": "matched",
        "scripts.eval_tree_traversal.leaf_metrics": {"recall": 1.0},
        "sparse.save_sparse_replay_plot": "plot",
    }


def test_script_modules_run_the_checkout_driver_with_the_hip_functions(tmp_path):
    stand_in = _write_stand_in(tmp_path / "checkout")
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([PKG, str(stand_in)]))
    for module, expected in (("scripts.export_selected_blocks", "packer=interfaces.packing"),
                             ("scripts.eval_tree_traversal", "traversal=selector.traversal")):
        res = subprocess.run([sys.executable, "-m", module], cwd=str(tmp_path), env=env,
                             capture_output=True, text=True, timeout=300)
        assert res.returncode == 0, res.stderr[-2000:]
        assert res.stdout.strip().splitlines()[-1] == expected


def test_without_a_checkout_only_this_build_exists(tmp_path):
    code = textwrap.dedent(f"""\
        import sys
        sys.path.insert(0, {PKG!r})
        from sparse import *
        import selector.tree, scripts.export_selected_blocks
        try:
            selector.tree.build_target_tree
        except AttributeError as e:
            print("attr:", e)
        try:
            import sparse.plotting
        except ModuleNotFoundError:
            print("plotting: absent")
        try:
            import runpy
            runpy.run_module("scripts.export_selected_blocks", run_name="__main__")
        except RuntimeError as e:
            print("main:", "not on sys.path" in str(e))
        print("config:", ResidualSummaryConfig().prototypes)
        """)
    res = _run(code, cwd=str(tmp_path))
    assert res.returncode == 0, res.stderr[-2000:]
    assert res.stdout.splitlines() == [
        "attr: module 'selector.tree' has no attribute 'build_target_tree'",
        "plotting: absent",
        "main: True",
        "config: 1",
    ]


def test_residual_summary_config_cli():
    """Known answers of the reference's tests/test_summary_config.py:12-41."""
    from sparse.config import (ResidualSummaryConfig, add_residual_summary_arguments,
                               residual_summary_config_from_args)
    parser = argparse.ArgumentParser()
    add_residual_summary_arguments(parser)
    assert residual_summary_config_from_args(parser.parse_args([])) == ResidualSummaryConfig()
    configured = residual_summary_config_from_args(parser.parse_args(
        ["--residual-summaries", "--summary-prototypes", "4", "--summary-mode", "learned",
         "--summary-checkpoint", "compressor.pt"]))
    assert configured == ResidualSummaryConfig(enabled=True, prototypes=4, mode="learned",
                                               checkpoint="compressor.pt")
    with pytest.raises(ValueError, match="requires --summary-checkpoint"):
        ResidualSummaryConfig(enabled=True, mode="learned")
    with pytest.raises(ValueError, match="summary prototypes must be one of"):
        ResidualSummaryConfig(prototypes=3)
    with pytest.raises(ValueError, match="summary mode must be one of"):
        ResidualSummaryConfig(mode="max")
    with pytest.raises(SystemExit):
        parser.parse_args(["--summary-prototypes", "3"])
    # A learned config that is not enabled needs no checkpoint; its kwargs feed the attention call.
    assert ResidualSummaryConfig(mode="learned").attention_kwargs() == {
        "residual_summaries": False, "summary_prototypes": 1, "summary_mode": "learned",
        "summary_checkpoint": None}
