"""How this package sits in front of a reference checkout on ``sys.path``.

The packages here (``sparse``, ``kernels``, ``selector``, ``teacher``,
``interfaces``, ``scripts``, ``benchmarks``) keep the reference's package and
module names, so that the reference's own callers -- its benchmark drivers,
replay scripts and Transformers registrations -- import the GPU path without
edits.  Put ``spruce-research_amd/`` ahead of the checkout and two mechanisms
keep the rest of the checkout importable:

* Every package here extends its ``__path__`` with the directories of the
  same name further down ``sys.path`` (``pkgutil.extend_path``).  A module this
  build does not ship -- ``sparse.plotting``, ``selector.recall``,
  ``teacher.prompt_replay``, ``scripts.route_overrides`` -- then loads from the
  checkout, while the modules this build does ship shadow theirs.
* A module here that replaces only part of a reference module (the key-tree
  builder of ``selector/tree.py`` but not its tree-KL training loss) gets a
  PEP 562 ``__getattr__`` from :func:`forward_missing`: a name it does not
  define is looked up in the checkout's file of the same name, loaded once
  under ``<module>__upstream``.  Its imports of shadowed modules resolve to
  this package, like every other caller's.

Without a checkout on the path, only the names this build defines exist and a
forwarded name raises ``AttributeError`` as for any missing attribute.
"""
import importlib.util
import os
import sys

_UPSTREAM = {}


def upstream_file(module_name, own_file):
    """The next file for ``module_name`` on its package's ``__path__`` that is not ``own_file``."""
    package, _, leaf = module_name.rpartition(".")
    parent = sys.modules.get(package)
    own_dir = os.path.dirname(os.path.realpath(own_file))
    for portion in getattr(parent, "__path__", ()):
        if os.path.realpath(portion) == own_dir:
            continue
        candidate = os.path.join(portion, leaf + ".py")
        if os.path.isfile(candidate):
            return candidate
    return None


def load_upstream(module_name, own_file):
    """The checkout's module that ``module_name`` here shadows, or None without a checkout."""
    if module_name in _UPSTREAM:
        return _UPSTREAM[module_name]
    path = upstream_file(module_name, own_file)
    module = None
    if path is not None:
        alias = module_name + "__upstream"
        spec = importlib.util.spec_from_file_location(alias, path)
        module = importlib.util.module_from_spec(spec)
        # Registered before it runs: dataclasses and pickling look the module up by name.
        sys.modules[alias] = module
        try:
            spec.loader.exec_module(module)
        except BaseException:
            del sys.modules[alias]
            raise
    _UPSTREAM[module_name] = module
    return module


def forward_missing(module_name, own_file):
    """A module ``__getattr__`` that takes names this module lacks from the checkout's module."""

    def __getattr__(name):
        if not (name.startswith("__") and name.endswith("__")):
            upstream = load_upstream(module_name, own_file)
            if upstream is not None and hasattr(upstream, name):
                return getattr(upstream, name)
        raise AttributeError(f"module {module_name!r} has no attribute {name!r}")

    return __getattr__


def run_upstream_main(module_name, own_file, overrides):
    """``python -m <module_name>`` for a script module this package replaces in part.

    Runs the checkout's ``main()`` after putting ``overrides`` (this package's
    functions, by name) in place of the checkout module's own, so the
    command-line driver computes through the GPU path.  Returns main's result.
    """
    upstream = load_upstream(module_name, own_file)
    if upstream is None or not hasattr(upstream, "main"):
        raise RuntimeError(
            f"{module_name} here replaces the library functions only; its command-line "
            "driver is the reference checkout's, which is not on sys.path")
    for name, value in overrides.items():
        setattr(upstream, name, value)
    return upstream.main()
