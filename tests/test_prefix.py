"""Prefix-block reuse (edgerag/cache/prefix.py), restating the reference's cases
(tests/test_cow.py:152-230) plus eviction; host only."""

from __future__ import annotations

import hashlib

from edgerag_amd.cache.allocator import BlockAllocator
from edgerag_amd.cache.prefix import ROOT_HASH, PrefixCache, chain_hash

BS = 8


def test_chain_hash_is_the_published_key_and_position_sensitive() -> None:
    expect = hashlib.sha256(b"root|1,2,3").hexdigest()[:32]
    assert chain_hash(ROOT_HASH, (1, 2, 3)) == expect
    a, b = chain_hash(ROOT_HASH, (1, 2, 3)), chain_hash(ROOT_HASH, (9, 9, 9))
    assert chain_hash(a, (4, 5, 6)) != chain_hash(b, (4, 5, 6))
    assert chain_hash(ROOT_HASH, (12, 3)) != chain_hash(ROOT_HASH, (1, 23))


def test_miss_reuse_and_partial_match() -> None:
    alloc = BlockAllocator(32, BS)
    cache = PrefixCache(alloc)
    assert cache.lookup(list(range(32))) == ([], 0) and cache.stats.hit_rate == 0.0
    tokens = list(range(24))
    blocks = alloc.allocate(3)
    assert cache.register(tokens, blocks) == 3
    assert cache.lookup(tokens) == (blocks, 24)
    matched, n = cache.lookup(list(range(16)) + [999] * 8)  # third block differs
    assert matched == blocks[:2] and n == 16
    alloc.check_invariants()


def test_trailing_partial_block_is_never_cached() -> None:
    alloc = BlockAllocator(16, BS)
    cache = PrefixCache(alloc)
    assert len(cache.block_hashes(list(range(20)))) == 2
    assert cache.register(list(range(20)), alloc.allocate(3)) == 2


def test_references_lookup_increfs_and_the_cache_keeps_its_own() -> None:
    alloc = BlockAllocator(16, BS)
    cache = PrefixCache(alloc)
    tokens = list(range(16))
    blocks = alloc.allocate(2)
    cache.register(tokens, blocks)
    before = [alloc.refcount(b) for b in blocks]
    matched, _ = cache.lookup(tokens)
    assert [alloc.refcount(b) for b in matched] == [r + 1 for r in before]
    alloc.free(matched)
    alloc.free(blocks)  # the first sequence finishes: the cache still holds them
    assert all(alloc.refcount(b) == 1 for b in blocks)
    assert cache.lookup(tokens)[0] == blocks


def test_lru_eviction_and_clear_release_the_references() -> None:
    alloc = BlockAllocator(16, BS)
    cache = PrefixCache(alloc, max_blocks=2)
    a, b = list(range(8)), list(range(100, 108))
    ba, bb = alloc.allocate(1), alloc.allocate(1)
    cache.register(a, ba)
    cache.register(b, bb)
    alloc.free(ba + bb)
    cache.lookup(a)  # a is now the most recent
    alloc.free(ba)
    c = list(range(200, 208))
    bc = alloc.allocate(1)
    assert cache.register(c, bc) == 1  # evicts b, the least recently used
    assert cache.stats.evictions == 1 and alloc.refcount(bb[0]) == 0
    assert cache.lookup(b) == ([], 0)
    alloc.free(cache.lookup(a)[0])
    alloc.free(bc)
    cache.clear()
    assert cache.num_cached == 0 and alloc.num_free == 16
    d = cache.to_dict()
    assert d["evictions"] == 1 and d["max_blocks"] == 2
