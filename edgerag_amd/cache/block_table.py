"""Logical token positions -> physical block ids, for one sequence (host bookkeeping).

Same contract as the reference ``BlockTable`` (``edgerag/cache/block_table.py:27-129``):
``blocks`` holds exactly ``ceil(num_tokens / block_size)`` ids; :meth:`append` grows capacity
before the length so a failed allocation leaves the table untouched; :meth:`fork` shares blocks;
:meth:`unshare` splits one shared block and leaves the content copy to the caller.

:meth:`slots` is the device-facing addition: the flat slot ids ``block * block_size + offset`` of
a position range, which is what the ``edgerag_kv_append`` kernel consumes.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import numpy as np

from edgerag_amd.cache.allocator import BlockAllocator


@dataclass
class BlockTable:
    allocator: BlockAllocator
    blocks: list[int] = field(default_factory=list)
    num_tokens: int = 0

    @property
    def block_size(self) -> int:
        return self.allocator.block_size

    @property
    def capacity(self) -> int:
        return len(self.blocks) * self.block_size

    @property
    def slack(self) -> int:
        return self.capacity - self.num_tokens

    def locate(self, position: int) -> tuple[int, int]:
        """``(physical block, offset)`` of a written position; IndexError past the written region."""
        if not 0 <= position < self.num_tokens:
            raise IndexError(
                f"position {position} outside the written region [0, {self.num_tokens}); "
                "reading past it would return a previous tenant's data"
            )
        return self.blocks[position // self.block_size], position % self.block_size

    def ensure_capacity(self, n_tokens: int) -> list[int]:
        """Grow so ``n_tokens`` fit; returns the freshly allocated blocks."""
        needed = self.allocator.blocks_needed(n_tokens)
        if needed <= len(self.blocks):
            return []
        fresh = self.allocator.allocate(needed - len(self.blocks))
        self.blocks.extend(fresh)
        return fresh

    def append(self, n_tokens: int = 1) -> list[int]:
        fresh = self.ensure_capacity(self.num_tokens + n_tokens)
        self.num_tokens += n_tokens
        return fresh

    def fork(self) -> BlockTable:
        self.allocator.incref(self.blocks)
        self.allocator.stats.forks += 1
        return BlockTable(self.allocator, list(self.blocks), self.num_tokens)

    def unshare(self, logical_block: int) -> tuple[int, int] | None:
        """Make ``logical_block`` private. ``(old, new)`` when a copy is needed, else None."""
        old = self.blocks[logical_block]
        new = self.allocator.copy_on_write(old)
        if new == old:
            return None
        self.blocks[logical_block] = new
        return old, new

    def writable_block_for(self, position: int) -> tuple[int, int, tuple[int, int] | None]:
        logical = position // self.block_size
        copied = self.unshare(logical)
        return self.blocks[logical], position % self.block_size, copied

    def slots(self, start: int, n: int) -> np.ndarray:
        """int32 slot ids of positions ``[start, start + n)``; they must be within capacity."""
        if start < 0 or start + n > self.capacity:
            raise IndexError(f"positions [{start}, {start + n}) exceed capacity {self.capacity}")
        pos = np.arange(start, start + n, dtype=np.int64)
        table = np.asarray(self.blocks, dtype=np.int64)
        return (table[pos // self.block_size] * self.block_size + pos % self.block_size).astype(
            np.int32
        )

    def free(self) -> int:
        reclaimed = self.allocator.free(self.blocks)
        self.blocks = []
        self.num_tokens = 0
        return reclaimed

    def to_dict(self) -> dict[str, Any]:
        return {
            "num_tokens": self.num_tokens,
            "num_blocks": len(self.blocks),
            "capacity": self.capacity,
            "slack": self.slack,
            "blocks": list(self.blocks),
        }
