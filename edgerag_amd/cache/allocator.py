"""Physical block pool with reference counts -- host bookkeeping only, no tensors.

Same contract as the reference allocator (``edgerag/cache/allocator.py:76-254``):

* a LIFO free list that hands out block 0 first and reuses the most recently freed block
  (``:98-100``, ``:168``);
* all-or-nothing :meth:`allocate` raising :class:`OutOfBlocksError` (``:150-174``);
* reference counts for copy-on-write sharing, :class:`DoubleFreeError` on a second free
  (``:176-196``), :meth:`copy_on_write` returning the block unchanged when it is private
  (``:218-236``);
* ``blocks_needed = ceil(n / block_size)`` (``:244-254``) and :meth:`check_invariants`
  (``:120-146``).

On MI355X the pool itself is one head-major tensor per layer in HBM; this object only decides
which block ids a sequence owns. The executor turns those ids into device block tables and slot
mappings once per step.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

#: Sentinel for "no physical block" in int32 block tables.
NO_BLOCK = -1


class AllocatorError(RuntimeError):
    """Misuse of the allocator: always a caller bug."""


class OutOfBlocksError(AllocatorError):
    """The pool cannot satisfy a request. An expected runtime condition (admission, preemption)."""


class DoubleFreeError(AllocatorError):
    """A block was released while already free; it would otherwise be handed out twice."""


@dataclass
class AllocatorStats:
    total_blocks: int
    block_size: int
    allocations: int = 0
    frees: int = 0
    forks: int = 0
    copy_on_writes: int = 0
    peak_used_blocks: int = 0
    oom_events: int = 0
    extra: dict[str, Any] = field(default_factory=dict)


class BlockAllocator:
    """Fixed-size block pool with reference counting and a LIFO free list."""

    def __init__(self, num_blocks: int, block_size: int) -> None:
        if num_blocks <= 0:
            raise ValueError(f"num_blocks must be positive, got {num_blocks}")
        if block_size <= 0:
            raise ValueError(f"block_size must be positive, got {block_size}")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self._refs = [0] * num_blocks
        # Top of the stack is the end of the list: block 0 sits on top initially.
        self._stack = list(reversed(range(num_blocks)))
        self.stats = AllocatorStats(total_blocks=num_blocks, block_size=block_size)

    # --- inspection -----------------------------------------------------------------------------

    @property
    def num_free(self) -> int:
        return len(self._stack)

    @property
    def num_used(self) -> int:
        return self.num_blocks - len(self._stack)

    @property
    def utilization(self) -> float:
        return self.num_used / self.num_blocks

    def refcount(self, block: int) -> int:
        return self._refs[block]

    def check_invariants(self) -> None:
        """Raise AllocatorError unless free list and reference counts agree exactly."""
        on_stack = set(self._stack)
        if len(on_stack) != len(self._stack):
            raise AllocatorError(
                f"free list holds duplicates ({len(self._stack)} entries, {len(on_stack)} distinct)"
            )
        for block, refs in enumerate(self._refs):
            free = block in on_stack
            if free and refs != 0:
                raise AllocatorError(f"block {block} is free but has refcount {refs}")
            if not free and refs <= 0:
                raise AllocatorError(f"block {block} is allocated but has refcount {refs}")
        if self.num_used + self.num_free != self.num_blocks:
            raise AllocatorError("conservation violated")

    # --- allocation -----------------------------------------------------------------------------

    def allocate(self, n_blocks: int = 1) -> list[int]:
        """Take ``n_blocks`` blocks at refcount 1, or none at all."""
        if n_blocks < 0:
            raise ValueError(f"cannot allocate {n_blocks} blocks")
        if n_blocks == 0:
            return []
        if n_blocks > len(self._stack):
            self.stats.oom_events += 1
            raise OutOfBlocksError(
                f"requested {n_blocks} blocks, only {self.num_free} free "
                f"({self.num_used}/{self.num_blocks} in use)"
            )
        taken = self._stack[-n_blocks:][::-1]
        del self._stack[-n_blocks:]
        for block in taken:
            self._refs[block] = 1
        self.stats.allocations += n_blocks
        self.stats.peak_used_blocks = max(self.stats.peak_used_blocks, self.num_used)
        return taken

    def free(self, blocks: list[int]) -> int:
        """Drop one reference per block; return how many blocks went back to the pool."""
        reclaimed = 0
        for block in blocks:
            self._validate(block)
            if self._refs[block] == 0:
                raise DoubleFreeError(
                    f"block {block} freed while already free; it would be handed to two "
                    "sequences at once"
                )
            self._refs[block] -= 1
            if self._refs[block] == 0:
                self._stack.append(block)
                reclaimed += 1
        self.stats.frees += len(blocks)
        return reclaimed

    def incref(self, blocks: list[int]) -> None:
        """Share blocks (fork). Rejects free blocks rather than resurrecting them."""
        for block in blocks:
            self._validate(block)
            if self._refs[block] == 0:
                raise AllocatorError(f"cannot incref free block {block}")
        for block in blocks:
            self._refs[block] += 1

    def is_shared(self, block: int) -> bool:
        self._validate(block)
        return self._refs[block] > 1

    def copy_on_write(self, block: int) -> int:
        """New private block replacing a shared one (caller copies contents); same id if private."""
        self._validate(block)
        if self._refs[block] == 0:
            raise AllocatorError(f"cannot copy-on-write free block {block}")
        if self._refs[block] == 1:
            return block
        fresh = self.allocate(1)[0]
        self._refs[block] -= 1
        self.stats.copy_on_writes += 1
        return fresh

    def _validate(self, block: int) -> None:
        if not 0 <= block < self.num_blocks:
            raise AllocatorError(f"block id {block} out of range [0, {self.num_blocks})")

    # --- arithmetic -------------------------------------------------------------------------------

    def blocks_needed(self, n_tokens: int) -> int:
        """``ceil(n_tokens / block_size)``: exact multiples get no spare block."""
        if n_tokens < 0:
            raise ValueError(f"negative token count {n_tokens}")
        return -(-n_tokens // self.block_size)

    def internal_fragmentation(self, sequence_lengths: list[int]) -> dict[str, float]:
        capacity = sum(self.blocks_needed(n) * self.block_size for n in sequence_lengths)
        wasted = capacity - sum(sequence_lengths)
        return {
            "wasted_tokens": float(wasted),
            "wasted_blocks_equiv": wasted / self.block_size,
            "waste_fraction": wasted / capacity if capacity else 0.0,
        }

    def to_dict(self) -> dict[str, Any]:
        s = self.stats
        return {
            "num_blocks": self.num_blocks,
            "block_size": self.block_size,
            "num_free": self.num_free,
            "num_used": self.num_used,
            "utilization": round(self.utilization, 4),
            "stats": {
                "allocations": s.allocations,
                "frees": s.frees,
                "forks": s.forks,
                "copy_on_writes": s.copy_on_writes,
                "peak_used_blocks": s.peak_used_blocks,
                "oom_events": s.oom_events,
            },
        }
