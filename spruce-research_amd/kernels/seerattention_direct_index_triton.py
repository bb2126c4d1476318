"""Reference module path kept for drop-in imports; the implementation is HIP.

Callers of the reference import ``KERNEL_VARIANTS``,
``direct_index_sparse_triton`` and ``kernel_runtime_metadata`` from this module
path (kernels/seerattention_direct_index_triton.py:17-23, 339-447).  The names
resolve to the gfx950 kernels in ``kernels.direct_index``; no Triton is used.
"""
from kernels.direct_index import (  # noqa: F401
    KERNEL_VARIANTS,
    direct_index_sparse_csr,
    direct_index_sparse_prefill as direct_index_sparse_triton,
    kernel_runtime_metadata,
)

__all__ = ["KERNEL_VARIANTS", "direct_index_sparse_triton", "kernel_runtime_metadata",
           "direct_index_sparse_csr"]
