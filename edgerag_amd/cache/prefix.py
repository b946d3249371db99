"""Reuse of already-computed prompt blocks across requests, indexed by chained content keys.

The index is a forest: each cached block is a node keyed by the hash of its parent's key and its
own token ids, so a node stands for the whole prefix that ends with it and can only match at its
own position (its keys were computed with RoPE at those positions).

* Only full blocks are indexed; a partial block is still being appended to.
* The index owns one pool reference per node, so the last sequence releasing a block cannot hand
  it to the allocator while the index still points at it. :meth:`PrefixCache.lookup` adds one
  more reference per matched block, owned by the caller.
* Eviction removes the least recently used *leaf*. Removing an inner node would strand its
  descendants (no lookup can reach them again, yet they keep pinning blocks); evicting leaves
  only keeps every cached node reachable. Leaves wait in a heap ordered by last use; entries whose
  node has since been touched, evicted or given children are skipped when popped.

The key format is the reference's (``edgerag/cache/prefix.py:36-48``), so keys computed on
either side agree: SHA-256 over the parent key, ``|`` and the comma-joined token ids, first 32 hex
digits; the chain starts from ``"root"``.
"""

from __future__ import annotations

import hashlib
import heapq
from dataclasses import dataclass
from typing import Iterator

from edgerag_amd.cache.allocator import BlockAllocator

#: Parent key of a prompt's first block.
ROOT_HASH = "root"


def chain_hash(parent: str, tokens: tuple[int, ...] | list[int]) -> str:
    """Key of the block holding ``tokens`` whose preceding prefix has key ``parent``."""
    digest = hashlib.sha256(f"{parent}|{','.join(map(str, tokens))}".encode())
    return digest.hexdigest()[:32]


@dataclass
class _Node:
    block: int
    parent: str | None  # None: a first block (parent is ROOT_HASH)
    children: int
    last_use: int


@dataclass
class PrefixCounters:
    queries: int = 0
    queries_hit: int = 0
    blocks_served: int = 0
    blocks_indexed: int = 0
    blocks_evicted: int = 0


class PrefixCache:
    def __init__(self, allocator: BlockAllocator, max_blocks: int | None = None) -> None:
        """``max_blocks`` bounds the blocks the index pins (default: a quarter of the pool)."""
        self.allocator = allocator
        self.max_blocks = max_blocks if max_blocks is not None else max(1, allocator.num_blocks // 4)
        if self.max_blocks < 1:
            raise ValueError("the prefix index must be allowed at least one block")
        self._nodes: dict[str, _Node] = {}
        self._leaves: list[tuple[int, str]] = []  # (last_use, key), lazily invalidated
        self._clock = 0
        self.counters = PrefixCounters()

    @property
    def num_cached(self) -> int:
        return len(self._nodes)

    def _keys(self, token_ids: list[int]) -> Iterator[tuple[str, str | None]]:
        """``(key, parent key)`` of each full block of ``token_ids``, generated lazily."""
        bs = self.allocator.block_size
        parent = ROOT_HASH
        for start in range(0, len(token_ids) - bs + 1, bs):
            key = chain_hash(parent, token_ids[start : start + bs])
            yield key, (None if parent == ROOT_HASH else parent)
            parent = key

    def block_hashes(self, token_ids: list[int]) -> list[str]:
        """Keys of every full block of ``token_ids``."""
        return [k for k, _ in self._keys(token_ids)]

    def _touch(self, key: str, node: _Node) -> None:
        self._clock += 1
        node.last_use = self._clock
        if node.children == 0:
            heapq.heappush(self._leaves, (node.last_use, key))
            if len(self._leaves) > 4 * len(self._nodes) + 64:  # drop stale entries
                self._leaves = [(n.last_use, k) for k, n in self._nodes.items() if not n.children]
                heapq.heapify(self._leaves)

    def lookup(self, token_ids: list[int], max_tokens: int | None = None) -> tuple[list[int], int]:
        """Blocks of the longest indexed prefix of ``token_ids`` (at most ``max_tokens`` tokens)
        and the number of tokens they hold. The caller owns one new reference per block."""
        self.counters.queries += 1
        bs = self.allocator.block_size
        limit = len(token_ids) if max_tokens is None else min(max_tokens, len(token_ids))
        found: list[int] = []
        for key, _ in self._keys(token_ids[: limit // bs * bs]):
            node = self._nodes.get(key)
            if node is None:
                break
            found.append(node.block)
            self._touch(key, node)
        if found:
            self.allocator.incref(found)
            self.counters.queries_hit += 1
            self.counters.blocks_served += len(found)
        return found, len(found) * bs

    def register(self, token_ids: list[int], blocks: list[int] | object) -> int:
        """Index the full blocks of a computed prompt (``blocks[i]`` holds block ``i`` of
        ``token_ids``); already-indexed prefixes are kept. The index takes its own reference on
        each new node; the caller keeps its own. Returns the nodes added."""
        blocks = [int(b) for b in blocks]
        added = 0
        for i, (key, parent) in enumerate(self._keys(token_ids)):
            if i >= len(blocks):
                break
            node = self._nodes.get(key)
            if node is not None:
                self._touch(key, node)
                continue
            if not self._make_room(protect=parent):
                break
            self.allocator.incref([blocks[i]])
            if parent is not None:
                self._nodes[parent].children += 1
            node = self._nodes[key] = _Node(blocks[i], parent, 0, 0)
            self._touch(key, node)
            added += 1
        self.counters.blocks_indexed += added
        return added

    def _make_room(self, protect: str | None) -> bool:
        """Evict least recently used leaves until one more node fits; never the node ``protect``
        (the parent about to receive a child). False if nothing can be evicted."""
        while len(self._nodes) >= self.max_blocks:
            victim = self._pop_leaf(protect)
            if victim is None:
                return False
            self._evict(victim)
        return True

    def _pop_leaf(self, protect: str | None) -> str | None:
        held = []
        found = None
        while self._leaves:
            stamp, key = heapq.heappop(self._leaves)
            node = self._nodes.get(key)
            if node is None or node.children or node.last_use != stamp:
                continue  # stale heap entry
            if key == protect:
                held.append((stamp, key))
                continue
            found = key
            break
        for item in held:
            heapq.heappush(self._leaves, item)
        return found

    def _evict(self, key: str) -> None:
        node = self._nodes.pop(key)
        self.allocator.free([node.block])
        self.counters.blocks_evicted += 1
        if node.parent is not None:
            parent = self._nodes[node.parent]
            parent.children -= 1
            if parent.children == 0:
                heapq.heappush(self._leaves, (parent.last_use, node.parent))

    def clear(self) -> None:
        """Drop every node and the index's references."""
        blocks = [n.block for n in self._nodes.values()]
        self._nodes.clear()
        self._leaves.clear()
        if blocks:
            self.allocator.free(blocks)

    def snapshot(self) -> dict:
        c = self.counters
        return {
            "indexed_blocks": self.num_cached, "limit_blocks": self.max_blocks,
            "queries": c.queries, "queries_hit": c.queries_hit,
            "hit_fraction": round(c.queries_hit / c.queries, 4) if c.queries else 0.0,
            "blocks_served": c.blocks_served, "blocks_indexed": c.blocks_indexed,
            "blocks_evicted": c.blocks_evicted,
        }
