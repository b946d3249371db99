"""The reference's block-table and executor-facing contracts, on this package's array-backed
table. CPU only.

The reference executor grows every request's table with ``cache.table.ensure_capacity(seq_len +
n)`` before each forward and then lets ``PagedKVCache.update`` advance the length on the first
layer (``edgerag/serve/executor.py:124-128``, ``:151-153``; ``edgerag/cache/paged.py:138-142``).
Its scheduler reads ``table.blocks`` as a list, assigns ``table.blocks = []`` and
``table.num_tokens = 0`` when it hands a preempted request's blocks to the swapper, and grows
through ``ensure_capacity`` (``edgerag/sched/scheduler.py:233-251``, ``:271-288``). The table
arithmetic below restates ``tests/test_paged.py:172-288`` case for case.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from edgerag_amd.cache.allocator import BlockAllocator, OutOfBlocksError
from edgerag_amd.cache.block_table import BlockTable
from edgerag_amd.cache.paged import PagedKVCache
from edgerag_amd.core.spec import ModelSpec

SPEC = ModelSpec(model_id="tiny", model_type="llama", n_layers=3, hidden_size=64, n_q_heads=4,
                 n_kv_heads=2, head_dim=16, vocab_size=64, max_position_embeddings=512,
                 rope_theta=10000.0, intermediate_size=128)


# --- table arithmetic (tests/test_paged.py:172-230) -----------------------------------------------


def test_locate_refuses_positions_past_the_written_region() -> None:
    table = BlockTable(allocator=BlockAllocator(8, 16))
    table.append(17)
    table.locate(16)
    for bad in (17, 31, 100):
        with pytest.raises(IndexError, match="outside the written region"):
            table.locate(bad)


@pytest.mark.parametrize(
    ("tokens", "block_size", "expected_blocks"),
    [(1, 16, 1), (16, 16, 1), (17, 16, 2), (32, 16, 2), (33, 16, 3), (8, 8, 1), (9, 8, 2)],
)
def test_table_holds_exactly_the_blocks_needed(tokens, block_size, expected_blocks) -> None:
    table = BlockTable(allocator=BlockAllocator(16, block_size))
    table.append(tokens)
    assert len(table.blocks) == expected_blocks
    assert table.num_tokens == tokens


def test_appending_one_token_past_a_full_block_allocates_exactly_one() -> None:
    table = BlockTable(allocator=BlockAllocator(8, 16))
    table.append(16)
    assert len(table.blocks) == 1
    fresh = table.append(1)
    assert len(fresh) == 1 and len(table.blocks) == 2


def test_slack_reports_internal_fragmentation() -> None:
    table = BlockTable(allocator=BlockAllocator(8, 16))
    table.append(17)
    assert table.capacity == 32 and table.slack == 15
    assert table.to_dict() == {"num_tokens": 17, "num_blocks": 2, "capacity": 32, "slack": 15,
                               "blocks": [0, 1]}
    frag = table.allocator.internal_fragmentation([17])
    assert frag["wasted_tokens"] == 15.0 and frag["waste_fraction"] == pytest.approx(15 / 32)
    assert table.allocator.internal_fragmentation([16, 32, 48])["wasted_tokens"] == 0.0


def test_failed_growth_leaves_the_table_untouched() -> None:
    table = BlockTable(allocator=BlockAllocator(2, 16))
    table.append(32)
    with pytest.raises(OutOfBlocksError):
        table.append(1)
    assert table.num_tokens == 32 and len(table.blocks) == 2
    with pytest.raises(OutOfBlocksError):
        table.ensure_capacity(33)
    assert len(table.blocks) == 2


def test_free_returns_blocks_and_resets() -> None:
    allocator = BlockAllocator(8, 16)
    table = BlockTable(allocator=allocator)
    table.append(40)
    assert allocator.num_used == 3
    assert table.free() == 3
    assert allocator.num_free == 8 and table.num_tokens == 0 and table.blocks == []
    allocator.check_invariants()


# --- fork / copy-on-write bookkeeping (tests/test_paged.py:233-288) -------------------------------


def test_fork_shares_blocks_without_copying() -> None:
    allocator = BlockAllocator(16, 16)
    parent = BlockTable(allocator=allocator)
    parent.append(32)
    used_before = allocator.num_used
    child = parent.fork()
    assert child.blocks == parent.blocks
    assert allocator.num_used == used_before
    assert all(allocator.refcount(b) == 2 for b in parent.blocks)
    assert allocator.stats.forks == 1
    allocator.check_invariants()


def test_writing_to_a_forked_block_splits_it() -> None:
    allocator = BlockAllocator(16, 16)
    parent = BlockTable(allocator=allocator)
    parent.append(16)
    child = parent.fork()
    block, offset, copied = child.writable_block_for(0)
    assert copied is not None and offset == 0
    old, new = copied
    assert block == new != old
    assert parent.blocks[0] == old
    assert allocator.refcount(old) == 1
    assert allocator.stats.copy_on_writes == 1
    allocator.check_invariants()


def test_writing_to_an_unshared_block_does_not_copy() -> None:
    allocator = BlockAllocator(16, 16)
    table = BlockTable(allocator=allocator)
    table.append(16)
    block, offset, copied = table.writable_block_for(5)
    assert copied is None and (block, offset) == (0, 5)
    assert allocator.stats.copy_on_writes == 0


def test_freeing_a_fork_leaves_the_parent_intact() -> None:
    allocator = BlockAllocator(16, 16)
    parent = BlockTable(allocator=allocator)
    parent.append(32)
    child = parent.fork()
    assert child.free() == 0
    assert all(allocator.refcount(b) == 1 for b in parent.blocks)
    assert parent.free() == 2
    assert allocator.num_free == 16
    allocator.check_invariants()


def test_allocator_report_keys() -> None:
    allocator = BlockAllocator(8, 16)
    table = BlockTable(allocator=allocator)
    table.append(20)
    table.fork().free()
    report = allocator.to_dict()
    assert report["num_used"] == 2 and report["num_free"] == 6
    assert report["stats"] == {"allocations": 2, "frees": 2, "forks": 1, "copy_on_writes": 0,
                               "peak_used_blocks": 2, "oom_events": 0}


# --- the reference executor's and scheduler's call sequences ------------------------------------


def _cache(allocator: BlockAllocator) -> PagedKVCache:
    return PagedKVCache(SPEC, allocator, torch.device("cpu"), torch.float32)


def test_reference_executor_sequence_grows_once_per_forward() -> None:
    """``ensure_capacity(seq_len + n)`` before the forward, then the first layer's growth (the
    host half of ``update``) takes no further block and advances the length by exactly ``n``; the
    slots of the new positions are ``blocks[p // 16] * 16 + p % 16``."""
    allocator = BlockAllocator(64, 16)
    cache = _cache(allocator)
    for n in (37, 27, 1, 1, 16, 1):  # a prefill in two chunks, decodes, a block-sized chunk
        before = cache.seq_len
        fresh = cache.table.ensure_capacity(cache.seq_len + n)
        assert len(fresh) == allocator.blocks_needed(before + n) - allocator.blocks_needed(before)
        used = allocator.num_used
        slots = cache.reserve(n)  # what update() does on the first layer, before its writes
        assert allocator.num_used == used, "the forward allocated again after ensure_capacity"
        assert cache.seq_len == before + n
        assert len(cache.table.blocks) == allocator.blocks_needed(cache.seq_len)
        pos = np.arange(before, before + n)
        ids = np.asarray(cache.table.blocks)
        np.testing.assert_array_equal(slots, ids[pos // 16] * 16 + pos % 16)
    allocator.check_invariants()


def test_reference_scheduler_preemption_hands_blocks_over() -> None:
    """The reference scheduler's swap hand-over: read the blocks as a list, empty the table by
    assignment, release later through the swapper; owner counts move only on that release."""
    allocator = BlockAllocator(32, 16)
    cache = _cache(allocator)
    cache.table.ensure_capacity(70)
    cache.table.append(70)
    blocks = list(cache.table.blocks)
    assert blocks == [0, 1, 2, 3, 4] and all(isinstance(b, int) for b in blocks)
    cache.table.blocks = []
    cache.table.num_tokens = 0
    assert cache.seq_len == 0 and cache.table.capacity == 0 and not cache.table.blocks
    assert allocator.num_used == 5  # still owned by the swap record
    assert allocator.free(blocks) == 5
    allocator.check_invariants()
    # a restored request gets its (new) blocks assigned back
    restored = allocator.allocate(5)
    cache.table.blocks = restored
    cache.table.num_tokens = 70
    assert cache.table.locate(69) == (restored[4], 5)


def test_reference_try_allocate_sequence() -> None:
    """``try_allocate``: ``ensure_capacity`` raises when short and leaves the table intact, then
    succeeds after blocks are freed (``sched/scheduler.py:271-288``)."""
    allocator = BlockAllocator(4, 16)
    hog = BlockTable(allocator=allocator)
    hog.append(48)
    cache = _cache(allocator)
    cache.table.append(10)
    with pytest.raises(OutOfBlocksError):
        cache.table.ensure_capacity(cache.seq_len + 20)
    assert cache.table.blocks == [3] and cache.seq_len == 10
    hog.free()
    assert cache.table.ensure_capacity(cache.seq_len + 20) == [2]
    assert cache.seq_len == 10
    allocator.check_invariants()
