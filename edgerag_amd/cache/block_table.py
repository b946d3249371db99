"""One sequence's logical-to-physical block map, kept as a growable int32 array, plus the batch
helpers that turn many maps into the step's device metadata in a few numpy operations.

A table holds ``len(blocks) == ceil(num_tokens / block_size)`` physical ids
(``edgerag/cache/block_table.py:27-129`` keeps the same count): logical position ``p`` lives in
block ``blocks[p // block_size]`` at offset ``p % block_size``, i.e. in pool slot
``blocks[p // block_size] * block_size + p % block_size``.

The methods keep the reference's names and contracts, so its executor and scheduler drive this
table unchanged:

* :meth:`ensure_capacity` takes blocks for a length without moving it; :meth:`append` takes the
  blocks for ``n`` more tokens before it moves the length, so a refused allocation leaves the
  table as it was (``block_table.py:62-79``);
* :meth:`fork` shares every block with a new table (one more owner each);
* :meth:`unshare` / :meth:`writable_block_for` give a shared block a private copy (the caller
  moves the contents); :meth:`free` drops every ownership;
* :meth:`locate` refuses positions that were never written (they hold a previous tenant's data);
* ``blocks`` reads as a list of ints and may be assigned; ``num_tokens`` is a plain attribute.

The ids live in a growable int32 array (:attr:`ids` is a view of it), which is what the batch
helpers read.

:func:`pack_tables` and :func:`step_slots` build a whole batch's ``[R, width]`` block-table matrix
and its slot mapping for the single per-step upload.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np

from edgerag_amd.cache.allocator import NO_BLOCK, BlockAllocator


class BlockTable:
    __slots__ = ("allocator", "_ids", "_n", "num_tokens")

    def __init__(self, allocator: BlockAllocator, blocks: Sequence[int] | np.ndarray = (),
                 num_tokens: int = 0) -> None:
        self.allocator = allocator
        self._ids = np.empty(8, dtype=np.int32)
        self._n = 0
        self.blocks = blocks
        self.num_tokens = int(num_tokens)

    # --- shape ------------------------------------------------------------------------------------

    @property
    def block_size(self) -> int:
        return self.allocator.block_size

    @property
    def ids(self) -> np.ndarray:
        """The physical ids, int32, logical order (a view: do not keep it across a change)."""
        return self._ids[: self._n]

    @property
    def blocks(self) -> list[int]:
        """The physical ids as a list of ints (a copy), the reference's field
        (``block_table.py:31``)."""
        return self._ids[: self._n].tolist()

    @blocks.setter
    def blocks(self, ids: Sequence[int] | np.ndarray) -> None:
        """Replace the mapping without touching owner counts, as assigning the reference's field
        does: its scheduler hands a preempted table's blocks to the swapper this way
        (``sched/scheduler.py:244-245``)."""
        arr = np.asarray(ids, dtype=np.int32).reshape(-1)
        if arr.size > self._ids.size:
            self._ids = np.empty(max(8, arr.size), dtype=np.int32)
        self._ids[: arr.size] = arr
        self._n = int(arr.size)

    @property
    def num_blocks(self) -> int:
        return self._n

    @property
    def capacity(self) -> int:
        return self._n * self.block_size

    @property
    def slack(self) -> int:
        return self.capacity - self.num_tokens

    # --- growth and release -------------------------------------------------------------------------

    def _push(self, fresh: list[int]) -> None:
        need = self._n + len(fresh)
        if need > self._ids.size:
            bigger = np.empty(max(need, 2 * self._ids.size), dtype=np.int32)
            bigger[: self._n] = self._ids[: self._n]
            self._ids = bigger
        self._ids[self._n : need] = fresh
        self._n = need

    def ensure_capacity(self, n_tokens: int) -> list[int]:
        """Hold enough blocks for ``n_tokens`` tokens without moving the length. Returns the
        fresh ids (none when the table is already big enough); a refused allocation raises
        :class:`OutOfBlocksError` and leaves the table as it was (``block_table.py:62-69``)."""
        missing = self.allocator.blocks_needed(n_tokens) - self._n
        if missing <= 0:
            return []
        fresh = self.allocator.allocate(missing)
        self._push(fresh)
        return fresh

    def append(self, n_tokens: int = 1) -> list[int]:
        """Count ``n_tokens`` more tokens as written, taking blocks first, so a refusal leaves
        the length unchanged (``block_table.py:71-79``). Returns the fresh ids."""
        if n_tokens < 0:
            raise ValueError(f"a table grows by >= 0 tokens, got {n_tokens}")
        fresh = self.ensure_capacity(self.num_tokens + n_tokens)
        self.num_tokens += n_tokens
        return fresh

    def shrink_to(self, n_tokens: int) -> int:
        """Undo growth: keep the first ``n_tokens`` tokens and release blocks past them. Returns
        the blocks released to the pool."""
        if not 0 <= n_tokens <= self.num_tokens:
            raise ValueError(f"cannot shrink {self.num_tokens} tokens to {n_tokens}")
        keep = self.allocator.blocks_needed(n_tokens)
        dropped = self._ids[keep : self._n].copy()
        self._n = keep
        self.num_tokens = n_tokens
        return self.allocator.free(dropped) if dropped.size else 0

    def free(self) -> int:
        """Drop this table's ownership of all its blocks and empty it. Returns how many blocks
        went back to the pool: fewer than the table held while another table shares some
        (``block_table.py:120-129``)."""
        freed = self.allocator.free(self.ids.copy()) if self._n else 0
        self._n = 0
        self.num_tokens = 0
        return freed

    def detach(self) -> tuple[list[int], int]:
        """Hand the blocks and token count over to a new owner (a swap-out record) and empty the
        table without releasing anything."""
        out = (self.blocks, self.num_tokens)
        self._n = 0
        self.num_tokens = 0
        return out

    def adopt(self, blocks: Sequence[int], num_tokens: int) -> None:
        """Take over already-owned ``blocks`` holding ``num_tokens`` tokens (a swap-in)."""
        if self._n:
            raise RuntimeError("only an empty table can adopt blocks")
        if len(blocks) != self.allocator.blocks_needed(num_tokens):
            raise ValueError(f"{len(blocks)} blocks cannot hold exactly {num_tokens} tokens")
        self._push(list(blocks))
        self.num_tokens = int(num_tokens)

    # --- sharing ----------------------------------------------------------------------------------

    def fork(self) -> BlockTable:
        """A second table over the same blocks (each gains an owner; no contents move)."""
        self.allocator.incref(self.ids)
        self.allocator.counters.forks += 1
        return BlockTable(self.allocator, self.ids.copy(), self.num_tokens)

    def unshare(self, logical_block: int) -> tuple[int, int] | None:
        """Make logical block ``logical_block`` owned by this table alone. Returns
        ``(shared id, private id)`` when a fresh block replaced it -- the caller then copies the
        contents -- and None when it already was private (``block_table.py:95-107``)."""
        if not 0 <= logical_block < self._n:
            raise IndexError(f"logical block {logical_block} outside a table of {self._n}")
        old = int(self._ids[logical_block])
        new = self.allocator.copy_on_write(old)
        if new == old:
            return None
        self._ids[logical_block] = new
        return old, new

    def writable_block_for(self, position: int) -> tuple[int, int, tuple[int, int] | None]:
        """``(physical block, offset, copied)`` for a write at ``position``, after making its
        block private (``copied`` as :meth:`unshare` returns it) (``block_table.py:109-118``)."""
        bs = self.block_size
        copied = self.unshare(position // bs)
        return int(self._ids[position // bs]), position % bs, copied

    # --- addressing -------------------------------------------------------------------------------

    def locate(self, position: int) -> tuple[int, int]:
        """``(physical block, offset)`` of a written position."""
        if not 0 <= position < self.num_tokens:
            raise IndexError(
                f"position {position} outside the written region [0, {self.num_tokens}); its "
                "slot may hold another sequence's keys"
            )
        bs = self.block_size
        return int(self._ids[position // bs]), position % bs

    def slots(self, start: int, n: int) -> np.ndarray:
        """int32 pool slots of positions ``[start, start + n)`` (within capacity)."""
        if start < 0 or n < 0 or start + n > self.capacity:
            raise IndexError(
                f"positions [{start}, {start + n}) fall outside capacity {self.capacity}"
            )
        bs = self.block_size
        if n == 1:  # the decode step: plain integer arithmetic
            return np.array([int(self._ids[start // bs]) * bs + start % bs], dtype=np.int32)
        pos = np.arange(start, start + n, dtype=np.int64)
        return (self._ids[pos // bs].astype(np.int64) * bs + pos % bs).astype(np.int32)

    def to_dict(self) -> dict:
        """The reference report's keys (``block_table.py:131-138``)."""
        return {"num_tokens": self.num_tokens, "num_blocks": self._n,
                "capacity": self.capacity, "slack": self.slack, "blocks": self.blocks}


def pack_tables(tables: Sequence[BlockTable], width: int | None = None) -> np.ndarray:
    """``[len(tables), width]`` int32 block-table matrix, rows padded with ``NO_BLOCK``."""
    width = max([t.num_blocks for t in tables] + [1]) if width is None else width
    out = np.full((len(tables), width), NO_BLOCK, dtype=np.int32)
    for r, t in enumerate(tables):
        if t.num_blocks > width:
            raise ValueError(f"table {r} has {t.num_blocks} blocks, wider than {width}")
        out[r, : t.num_blocks] = t.ids
    return out


def step_slots(tables: Sequence[BlockTable], counts: Sequence[int]) -> np.ndarray:
    """Slot mapping of a packed step: for each table, its last ``counts[r]`` written positions
    (the tokens this step appends), concatenated in table order."""
    parts = [t.slots(t.num_tokens - c, c) for t, c in zip(tables, counts, strict=True)]
    return np.concatenate(parts) if parts else np.zeros(0, dtype=np.int32)
