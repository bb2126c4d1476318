"""Sparse prefill attention (HIP-backed drop-in for the reference's sparse package).

The package exports the reference's names (sparse/__init__.py:8-29 there).
``save_sparse_replay_plot`` is the reference's plotting helper, which this
build does not replace: it is imported from the checkout's ``sparse.plotting``
when first used, so the attention path does not need matplotlib (nor a
checkout: it is left out of ``__all__`` so that a star import never needs it).
"""
from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)

from sparse.attention import (  # noqa: E402
    SPARSE_PREFILL_ATTENTION,
    register_sparse_prefill_attention,
    sparse_prefill_attention_forward,
)
from sparse.config import ResidualSummaryConfig  # noqa: E402
from sparse.summaries import (  # noqa: E402
    KVSummaryTable,
    build_kv_summary_table,
    residual_attention_density,
)

__all__ = [
    "SPARSE_PREFILL_ATTENTION",
    "register_sparse_prefill_attention",
    "ResidualSummaryConfig",
    "KVSummaryTable",
    "build_kv_summary_table",
    "residual_attention_density",
    "sparse_prefill_attention_forward",
]


def __getattr__(name):
    if name == "save_sparse_replay_plot":
        from sparse.plotting import save_sparse_replay_plot
        return save_sparse_replay_plot
    raise AttributeError(f"module 'sparse' has no attribute {name!r}")
