"""Reference module path kept for drop-in imports; the implementation is HIP.

``block_sparse_triton(q, k, v, block_mask, scale, block_size=64)``
(kernels/seerattention_triton.py:71-90) resolves to the gfx950 block-mask
kernel in ``kernels.block_mask``; no Triton is used.
"""
from kernels.block_mask import block_sparse_prefill as block_sparse_triton  # noqa: F401

__all__ = ["block_sparse_triton"]
