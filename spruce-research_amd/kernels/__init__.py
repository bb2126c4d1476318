"""GPU kernels and adapters for SPRUCE sparse prefill (gfx950 HIP backend).

Same public names as the reference package (kernels/__init__.py:3-17).
"""
from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)

from kernels.sparse_prefill import (
    SPRUCE_HIP_SPARSE_PREFILL,
    SPRUCE_TRITON_SPARSE_PREFILL,
    register_triton_sparse_prefill_attention,
    selected_blocks_to_block_mask,
    selected_blocks_to_head_indices,
    triton_sparse_prefill_attention_forward,
)

__all__ = [
    "SPRUCE_HIP_SPARSE_PREFILL",
    "SPRUCE_TRITON_SPARSE_PREFILL",
    "register_triton_sparse_prefill_attention",
    "selected_blocks_to_block_mask",
    "selected_blocks_to_head_indices",
    "triton_sparse_prefill_attention_forward",
]
