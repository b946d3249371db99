"""Block pool accounting for the shared paged KV arena: which of the arena's blocks are taken,
and by how many owners. Host-side only; the arena itself is the per-layer head-major pools in HBM.

The state is two int32 arrays rather than Python lists, because what the device needs every step
is arrays: block tables and slot mappings are assembled with numpy and uploaded in one copy.

* ``_owners[b]`` -- how many holders (sequences, the prefix cache) reference block ``b``;
  0 means free.
* ``_stack[:_top]`` -- the free blocks, the next one to hand out on top. The stack starts as
  ``[n-1, ..., 1, 0]``, so a fresh pool hands out 0, 1, 2, ... and a released block is the next
  one reused (most recently released first).

Behaviour a caller of the reference allocator relies on (``edgerag/cache/allocator.py``):

* ``allocate(n)`` is all or nothing and raises :class:`OutOfBlocksError` when short
  (``:150-174``); the ids come out in the order above (``:98-100``, ``:168``);
* ``blocks_needed(n) = ceil(n / block_size)``, so an exact multiple gets no spare block
  (``:244-254``);
* releasing a free block raises :class:`DoubleFreeError`; sharing (``incref``) refuses free
  blocks; ``copy_on_write`` returns the block itself when it has one owner, otherwise a fresh
  block, moving one ownership over (``:176-236``).

Unlike the reference, a call that fails validation changes nothing: every id of a ``free`` or
``incref`` call is checked before any count moves.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Iterable

import numpy as np

#: Block-table entry for "no physical block" (int32 tables on the device).
NO_BLOCK = -1


class AllocatorError(RuntimeError):
    """The pool was used incorrectly (a bug in the caller, never a capacity condition)."""


class OutOfBlocksError(AllocatorError):
    """Not enough free blocks: an expected condition that admission or preemption handles."""


class DoubleFreeError(AllocatorError):
    """A block was released more times than it was owned."""


@dataclass
class PoolCounters:
    """Monotone event counts of one pool (for logs and the serving report)."""

    blocks_handed_out: int = 0
    blocks_released: int = 0
    shares: int = 0
    forks: int = 0
    private_copies: int = 0
    refusals: int = 0
    high_water: int = 0

    # The reference's ``AllocatorStats`` names for the same counts (``allocator.py:58-73``), read
    # by its tests and reports.
    @property
    def allocations(self) -> int:
        return self.blocks_handed_out

    @property
    def frees(self) -> int:
        return self.blocks_released

    @property
    def copy_on_writes(self) -> int:
        return self.private_copies

    @property
    def peak_used_blocks(self) -> int:
        return self.high_water

    @property
    def oom_events(self) -> int:
        return self.refusals


def _ids(blocks: Iterable[int] | np.ndarray) -> np.ndarray:
    return np.asarray(blocks if isinstance(blocks, np.ndarray) else list(blocks), dtype=np.int64)


class BlockAllocator:
    """A fixed arena of ``num_blocks`` blocks of ``block_size`` tokens with owner counts."""

    def __init__(self, num_blocks: int, block_size: int) -> None:
        if num_blocks < 1 or block_size < 1:
            raise ValueError(
                f"a block pool needs at least one block of at least one token "
                f"(got {num_blocks} blocks of {block_size})"
            )
        self.num_blocks = int(num_blocks)
        self.block_size = int(block_size)
        self._owners = np.zeros(self.num_blocks, dtype=np.int32)
        # Owners past the first, summed over blocks: 0 when nothing is shared, which lets the
        # per-step copy-on-write checks skip the owner array.
        self._extra_owners = 0
        self._stack = np.arange(self.num_blocks - 1, -1, -1, dtype=np.int32)
        self._top = self.num_blocks
        self.counters = PoolCounters()

    @property
    def stats(self) -> PoolCounters:
        """The event counts under the reference's attribute name (``allocator.py:104``)."""
        return self.counters

    # --- occupancy ------------------------------------------------------------------------------

    @property
    def num_free(self) -> int:
        return self._top

    @property
    def num_used(self) -> int:
        return self.num_blocks - self._top

    @property
    def utilization(self) -> float:
        return self.num_used / self.num_blocks

    def refcount(self, block: int) -> int:
        self._check_id(block)
        return int(self._owners[block])

    def is_shared(self, block: int) -> bool:
        return self.refcount(block) > 1

    def blocks_needed(self, n_tokens: int) -> int:
        """Blocks that hold ``n_tokens`` tokens: ``ceil(n_tokens / block_size)``."""
        if n_tokens < 0:
            raise ValueError(f"token count must be >= 0, got {n_tokens}")
        return (n_tokens + self.block_size - 1) // self.block_size

    # --- ownership changes ------------------------------------------------------------------------

    def allocate(self, n_blocks: int = 1) -> list[int]:
        """Hand out ``n_blocks`` free blocks, each with one owner; raise without change if short."""
        if n_blocks < 0:
            raise ValueError(f"block count must be >= 0, got {n_blocks}")
        if n_blocks > self._top:
            self.counters.refusals += 1
            raise OutOfBlocksError(
                f"pool exhausted: {n_blocks} blocks wanted, {self._top} of {self.num_blocks} free"
            )
        if n_blocks == 0:
            return []
        out = self._stack[self._top - n_blocks : self._top][::-1].copy()
        self._top -= n_blocks
        self._owners[out] = 1
        self.counters.blocks_handed_out += n_blocks
        self.counters.high_water = max(self.counters.high_water, self.num_used)
        return out.tolist()

    def free(self, blocks: Iterable[int] | np.ndarray) -> int:
        """Drop one ownership of each listed block (a block may be listed once per ownership);
        blocks left with no owner go back on the stack in list order. Returns how many did."""
        ids = _ids(blocks)
        if ids.size == 0:
            return 0
        self._check_range(ids)
        uniq, counts = np.unique(ids, return_counts=True)
        short = uniq[self._owners[uniq] < counts]
        if short.size:
            raise DoubleFreeError(
                f"release of block {int(short[0])} exceeds its {int(self._owners[short[0]])} "
                "owner(s): the block would be handed out twice"
            )
        np.subtract.at(self._owners, ids, 1)
        if uniq.size == ids.size:
            back = ids[self._owners[ids] == 0]
        else:  # a block listed several times goes back at its last listing
            last = {int(b): i for i, b in enumerate(ids.tolist())}
            back = np.array([b for b, i in sorted(last.items(), key=lambda kv: kv[1])
                             if self._owners[b] == 0], dtype=np.int64)
        self._stack[self._top : self._top + back.size] = back
        self._top += back.size
        # Every listing but a block's last (the one that frees it) dropped an extra owner.
        self._extra_owners -= int(ids.size - back.size)
        self.counters.blocks_released += int(ids.size)
        return int(back.size)

    def incref(self, blocks: Iterable[int] | np.ndarray) -> None:
        """Add one owner to each listed block (sharing); every block must already be owned."""
        ids = _ids(blocks)
        if ids.size == 0:
            return
        self._check_range(ids)
        unowned = ids[self._owners[ids] == 0]
        if unowned.size:
            raise AllocatorError(
                f"block {int(unowned[0])} is free: only owned blocks can be shared"
            )
        np.add.at(self._owners, ids, 1)
        self._extra_owners += int(ids.size)
        self.counters.shares += int(ids.size)

    def copy_on_write(self, block: int) -> int:
        """A block the caller may write: ``block`` itself if it has one owner, else a fresh block
        that takes over the caller's ownership (the caller copies the contents)."""
        self._check_id(block)
        owners = int(self._owners[block])
        if owners == 0:
            raise AllocatorError(f"block {block} is free: there is nothing to write into")
        if owners == 1:
            return int(block)
        fresh = self.allocate(1)[0]
        self._owners[block] -= 1
        self._extra_owners -= 1
        self.counters.private_copies += 1
        return fresh

    # --- checks -----------------------------------------------------------------------------------

    def _check_id(self, block: int) -> None:
        if not 0 <= block < self.num_blocks:
            raise AllocatorError(f"block {block} is not in this pool of {self.num_blocks}")

    def shared_count(self, blocks: np.ndarray) -> int:
        """How many of ``blocks`` (valid ids) have more than one owner."""
        if not self._extra_owners or not len(blocks):
            return 0
        return int(np.count_nonzero(self._owners[blocks] > 1))

    def _check_range(self, ids: np.ndarray) -> None:
        bad = ids[(ids < 0) | (ids >= self.num_blocks)]
        if bad.size:
            raise AllocatorError(f"block {int(bad[0])} is not in this pool of {self.num_blocks}")

    def check_invariants(self) -> None:
        """Raise :class:`AllocatorError` unless the stack and the owner counts agree: the stack
        holds distinct blocks, exactly the ones with no owner, and the running count of shared
        ownerships matches the owner counts."""
        free = self._stack[: self._top]
        if np.unique(free).size != free.size:
            raise AllocatorError("free stack lists a block twice")
        marked = np.zeros(self.num_blocks, dtype=bool)
        marked[free] = True
        if np.any(self._owners[marked] != 0):
            raise AllocatorError("a block on the free stack still has owners")
        if np.any(self._owners[~marked] <= 0):
            raise AllocatorError("a block off the free stack has no owner")
        extra = int(np.maximum(self._owners - 1, 0).sum())
        if extra != self._extra_owners:
            raise AllocatorError(f"{extra} owners past the first, the count says "
                                 f"{self._extra_owners}")

    def internal_fragmentation(self, sequence_lengths: Iterable[int]) -> dict[str, float]:
        """Slack of sequences of the given lengths: the unused tail of each one's last block
        (``allocator.py:256-274``)."""
        lengths = np.asarray(list(sequence_lengths), dtype=np.int64)
        held = (lengths + self.block_size - 1) // self.block_size * self.block_size
        wasted, capacity = float((held - lengths).sum()), float(held.sum())
        return {"wasted_tokens": wasted, "wasted_blocks_equiv": wasted / self.block_size,
                "waste_fraction": wasted / capacity if capacity else 0.0}

    def to_dict(self) -> dict:
        """Occupancy and event counts under the reference report's keys
        (``allocator.py:276-291``)."""
        c = self.counters
        return {
            "num_blocks": self.num_blocks, "block_size": self.block_size,
            "num_free": self.num_free, "num_used": self.num_used,
            "utilization": round(self.utilization, 4),
            "stats": {"allocations": c.allocations, "frees": c.frees, "forks": c.forks,
                      "copy_on_writes": c.copy_on_writes,
                      "peak_used_blocks": c.peak_used_blocks, "oom_events": c.oom_events},
        }

    def snapshot(self) -> dict:
        """Occupancy and event counts, for logs and the serving report."""
        c = self.counters
        return {
            "blocks": {"total": self.num_blocks, "free": self.num_free, "used": self.num_used,
                       "block_size": self.block_size},
            "events": {"handed_out": c.blocks_handed_out, "released": c.blocks_released,
                       "shared": c.shares, "forks": c.forks,
                       "private_copies": c.private_copies,
                       "refusals": c.refusals, "high_water": c.high_water},
        }
