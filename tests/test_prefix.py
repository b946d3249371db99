"""Prefix-block reuse (host only): the reference's key format and cases (tests/test_cow.py:152-230
in the reference), plus this index's own eviction rule -- least recently used *leaves* first, so
every indexed block stays reachable from the root."""

from __future__ import annotations

import hashlib

from edgerag_amd.cache.allocator import BlockAllocator
from edgerag_amd.cache.prefix import ROOT_HASH, PrefixCache, chain_hash

BS = 8


def test_chain_hash_is_the_published_key_and_position_sensitive() -> None:
    expect = hashlib.sha256(b"root|1,2,3").hexdigest()[:32]
    assert chain_hash(ROOT_HASH, (1, 2, 3)) == expect
    parent = hashlib.sha256(b"root|9,9").hexdigest()[:32]
    assert chain_hash(parent, [4, 5]) == hashlib.sha256(f"{parent}|4,5".encode()).hexdigest()[:32]
    a, b = chain_hash(ROOT_HASH, (1, 2, 3)), chain_hash(ROOT_HASH, (9, 9, 9))
    assert chain_hash(a, (4, 5, 6)) != chain_hash(b, (4, 5, 6))
    assert chain_hash(ROOT_HASH, (12, 3)) != chain_hash(ROOT_HASH, (1, 23))


def test_miss_reuse_and_partial_match() -> None:
    alloc = BlockAllocator(32, BS)
    cache = PrefixCache(alloc)
    assert cache.lookup(list(range(32))) == ([], 0)
    tokens = list(range(24))
    blocks = alloc.allocate(3)
    assert cache.register(tokens, blocks) == 3
    assert cache.lookup(tokens) == (blocks, 24)
    matched, n = cache.lookup(list(range(16)) + [999] * 8)  # third block differs
    assert matched == blocks[:2] and n == 16
    assert cache.lookup(tokens, max_tokens=23) == (blocks[:2], 16)  # whole blocks only
    assert cache.snapshot()["queries_hit"] == 3
    alloc.check_invariants()


def test_trailing_partial_block_is_never_indexed() -> None:
    alloc = BlockAllocator(16, BS)
    cache = PrefixCache(alloc)
    assert len(cache.block_hashes(list(range(20)))) == 2
    assert cache.register(list(range(20)), alloc.allocate(3)) == 2


def test_references_lookup_increfs_and_the_index_keeps_its_own() -> None:
    alloc = BlockAllocator(16, BS)
    cache = PrefixCache(alloc)
    tokens = list(range(16))
    blocks = alloc.allocate(2)
    cache.register(tokens, blocks)
    before = [alloc.refcount(b) for b in blocks]
    matched, _ = cache.lookup(tokens)
    assert [alloc.refcount(b) for b in matched] == [r + 1 for r in before]
    alloc.free(matched)
    alloc.free(blocks)  # the first sequence finishes: the index still holds them
    assert all(alloc.refcount(b) == 1 for b in blocks)
    assert cache.lookup(tokens)[0] == blocks


def test_eviction_takes_least_recently_used_leaves_and_keeps_chains_whole() -> None:
    """Two prompts share their first block. With room for 3 nodes, indexing a third prompt
    evicts the least recently used leaf -- never the shared first block, whose child would
    become unreachable."""
    alloc = BlockAllocator(32, BS)
    cache = PrefixCache(alloc, max_blocks=3)
    shared = list(range(8))
    a, b = shared + list(range(100, 108)), shared + list(range(200, 208))
    ba = alloc.allocate(2)
    cache.register(a, ba)
    bb = [ba[0]] + alloc.allocate(1)
    cache.register(b, bb)  # reuses node 0, adds b's second block
    assert cache.num_cached == 3
    cache.lookup(a)  # a's leaf is now the most recent; b's leaf is the LRU leaf
    alloc.free(cache.lookup(a)[0])
    c = list(range(300, 308))
    bc = alloc.allocate(1)
    assert cache.register(c, bc) == 1
    assert cache.snapshot()["blocks_evicted"] == 1
    assert cache.lookup(b)[1] == 8  # b's second block is gone, the shared first block is not
    assert cache.lookup(a)[1] == 16
    alloc.check_invariants()


def test_clear_releases_every_reference() -> None:
    alloc = BlockAllocator(16, BS)
    cache = PrefixCache(alloc, max_blocks=4)
    blocks = alloc.allocate(2)
    cache.register(list(range(16)), blocks)
    alloc.free(blocks)
    cache.clear()
    assert cache.num_cached == 0 and alloc.num_free == 16
