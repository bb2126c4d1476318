"""Block pooling of attention maps and the rollup pyramid (teacher/pool.py:3-39).

Tensor-library code on whatever device the input lives on; the HIP teacher
path produces pooled mass directly (teacher.chunked_extract.chunked_pool), and
these functions give the pyramid above it and the eager full-map check.
"""
import torch
import torch.nn.functional as F


def pool_attention(attn_layer, block_size):
    """[b, h, q_len, k_len] -> [b, h, q_blocks, k_blocks]: sums of each block (zero-padded tails)."""
    b, h, q_len, k_len = attn_layer.shape
    qb = (q_len + block_size - 1) // block_size
    kb = (k_len + block_size - 1) // block_size
    x = F.pad(attn_layer, (0, kb * block_size - k_len, 0, qb * block_size - q_len))
    return x.reshape(b, h, qb, block_size, kb, block_size).sum(dim=(3, 5))


def rollup(pooled):
    """Leaf-first list of levels; each parent cell is the sum of its 2x2 children.
    Stops once either block dimension is odd or below 2."""
    levels = [pooled]
    cur = pooled
    while cur.shape[-1] >= 2 and cur.shape[-2] >= 2 and cur.shape[-1] % 2 == 0 and cur.shape[-2] % 2 == 0:
        b, h, qb, kb = cur.shape
        cur = cur.reshape(b, h, qb // 2, 2, kb // 2, 2).sum(dim=(3, 5))
        levels.append(cur)
    return levels
