"""Oracle for the paged KV pool: slot-mapped write and gather (test infrastructure only).

Restates ``PagedKVCache._write`` (``edgerag/cache/paged.py:186-206``) and ``_gather_pool``
(``edgerag/cache/paged.py:229-238``) in torch CPU, plus the block-table arithmetic of
``BlockTable`` / ``BlockAllocator.blocks_needed`` (``edgerag/cache/block_table.py:48-79``,
``edgerag/cache/allocator.py:244-254``).
"""

from __future__ import annotations

import torch


def blocks_needed(n_tokens: int, block_size: int) -> int:
    """``ceil(n / bs)`` -- allocator.py:244-254."""
    return (n_tokens + block_size - 1) // block_size


def slot_mapping(block_ids: list[int], start: int, n_new: int, block_size: int) -> torch.Tensor:
    """Flat slots of positions ``[start, start+n_new)``: paged.py:198-204 as one index.

    ``block_of = block_ids[pos // bs]``, ``offset_of = pos % bs`` (paged.py:201-203), flattened
    into the ``(kv_heads, num_blocks * bs, head_dim)`` view as ``block_of * bs + offset_of``.
    """
    positions = torch.arange(start, start + n_new)
    table = torch.tensor(block_ids, dtype=torch.long)
    return table[positions // block_size] * block_size + positions % block_size


def write_slots(
    pool: torch.Tensor, source: torch.Tensor, block_ids: list[int], start: int
) -> None:
    """``pool[:, block_of, offset_of] = source[0].to(pool.dtype)`` -- paged.py:186-206.

    ``source`` is ``(1, kv_heads, n_new, head_dim)``; the pool is head-major
    ``(kv_heads, num_blocks, block_size, head_dim)``.
    """
    n_new = source.shape[2]
    block_size = pool.shape[2]
    positions = torch.arange(start, start + n_new)
    table = torch.tensor(block_ids, dtype=torch.long)
    block_of = table[positions // block_size]
    offset_of = positions % block_size
    pool[:, block_of, offset_of] = source[0].to(pool.dtype)


def gather_pool(pool: torch.Tensor, block_ids: list[int], seq_len: int) -> torch.Tensor:
    """``pool[:, ids].reshape(H, -1, d)[:, :seq_len]`` -- paged.py:229-238 (P-01 slice)."""
    n_kv_heads, _, _, head_dim = pool.shape
    if not block_ids:
        return torch.zeros((n_kv_heads, 0, head_dim), dtype=pool.dtype)
    blocks = pool[:, torch.tensor(block_ids, dtype=torch.long)]
    return blocks.reshape(n_kv_heads, -1, head_dim)[:, :seq_len]


def write_slots_bruteforce(
    pool: torch.Tensor, source: torch.Tensor, block_ids: list[int], start: int
) -> None:
    """Per-token loop over ``BlockTable.locate`` (block_table.py:48-60): the tiny-case pin."""
    block_size = pool.shape[2]
    for i in range(source.shape[2]):
        pos = start + i
        block, offset = block_ids[pos // block_size], pos % block_size
        for h in range(pool.shape[0]):
            pool[h, block, offset] = source[0, h, i].to(pool.dtype)
