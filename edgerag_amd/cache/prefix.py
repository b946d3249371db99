"""Prefix-block reuse by content hash (``edgerag/cache/prefix.py``, ``PrefixCache`` ``:64-172``).

A request hashes its prompt block by block; the leading run of blocks that an earlier request
already computed is handed over (its KV is reused, its prefill skipped) instead of recomputed.

* Only full blocks are cached: a partial block would be appended to at once (copy-on-write for
  nothing).
* A block's key chains the hashes of every block before it (``chain_hash``), so a block only ever
  matches at its own position: reused keys carry RoPE for the positions they were computed at.
* The cache owns one allocator reference per cached block, so a block cannot be freed by its
  last sequence and recycled under a live entry; ``lookup`` increfs what it returns (the caller
  owns those references). ``max_blocks`` (default a quarter of the pool) bounds what the cache
  pins; the least recently used entry is evicted first.

Host-only: the pools are untouched; the KV of a reused block is already on the device.
"""

from __future__ import annotations

import hashlib
from collections import OrderedDict
from dataclasses import dataclass
from typing import Any

from edgerag_amd.cache.allocator import BlockAllocator

#: Seed of every chain: the "empty prefix" parent.
ROOT_HASH = "root"


def chain_hash(parent: str, tokens: tuple[int, ...]) -> str:
    """Key of a block: SHA-256 of the parent key, ``|`` and the comma-joined token ids, first 32
    hex digits (the reference's key, ``edgerag/cache/prefix.py:36-48``)."""
    h = hashlib.sha256(parent.encode())
    h.update(b"|")
    h.update(",".join(str(t) for t in tokens).encode())
    return h.hexdigest()[:32]


@dataclass
class PrefixStats:
    lookups: int = 0
    hits: int = 0
    blocks_reused: int = 0
    tokens_reused: int = 0
    evictions: int = 0

    @property
    def hit_rate(self) -> float:
        return self.hits / self.lookups if self.lookups else 0.0


class PrefixCache:
    """Chained block hashes → physical blocks, LRU-bounded."""

    def __init__(self, allocator: BlockAllocator, max_blocks: int | None = None) -> None:
        self.allocator = allocator
        self.max_blocks = max_blocks if max_blocks is not None else max(1, allocator.num_blocks // 4)
        self._entries: OrderedDict[str, int] = OrderedDict()
        self.stats = PrefixStats()

    @property
    def num_cached(self) -> int:
        return len(self._entries)

    def block_hashes(self, token_ids: list[int]) -> list[tuple[str, tuple[int, ...]]]:
        """``(key, tokens)`` of each full block of ``token_ids``, chained from ``ROOT_HASH``."""
        bs = self.allocator.block_size
        out: list[tuple[str, tuple[int, ...]]] = []
        key = ROOT_HASH
        for start in range(0, len(token_ids) - bs + 1, bs):
            chunk = tuple(token_ids[start:start + bs])
            key = chain_hash(key, chunk)
            out.append((key, chunk))
        return out

    def lookup(self, token_ids: list[int]) -> tuple[list[int], int]:
        """Longest cached prefix: ``(blocks, tokens matched)``, stopping at the first miss. The
        returned blocks are increfed for the caller."""
        self.stats.lookups += 1
        matched: list[int] = []
        for key, _ in self.block_hashes(token_ids):
            block = self._entries.get(key)
            if block is None:
                break
            self._entries.move_to_end(key)
            matched.append(block)
        if not matched:
            return [], 0
        self.allocator.incref(matched)
        tokens = len(matched) * self.allocator.block_size
        self.stats.hits += 1
        self.stats.blocks_reused += len(matched)
        self.stats.tokens_reused += tokens
        return matched, tokens

    def register(self, token_ids: list[int], blocks: list[int]) -> int:
        """Cache the full blocks of a finished prefill (the cache takes its own reference on each;
        the caller keeps and frees its own). Returns the entries added."""
        added = 0
        for i, (key, _) in enumerate(self.block_hashes(token_ids)):
            if i >= len(blocks) or key in self._entries:
                continue
            self._evict_if_needed()
            if self.num_cached >= self.max_blocks:
                break
            self.allocator.incref([blocks[i]])
            self._entries[key] = blocks[i]
            added += 1
        return added

    def _evict_if_needed(self) -> None:
        while self._entries and self.num_cached >= self.max_blocks:
            _, block = self._entries.popitem(last=False)
            self.allocator.free([block])
            self.stats.evictions += 1

    def clear(self) -> None:
        """Drop every entry and its reference."""
        for block in self._entries.values():
            self.allocator.free([block])
        self._entries.clear()

    def to_dict(self) -> dict[str, Any]:
        return {
            "num_cached": self.num_cached,
            "max_blocks": self.max_blocks,
            "lookups": self.stats.lookups,
            "hits": self.stats.hits,
            "hit_rate": round(self.stats.hit_rate, 4),
            "blocks_reused": self.stats.blocks_reused,
            "tokens_reused": self.stats.tokens_reused,
            "evictions": self.stats.evictions,
        }
