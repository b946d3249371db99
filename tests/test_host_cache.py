"""Host bookkeeping of the paged pool: the allocator, block tables and the executor's
all-or-nothing step reservation. CPU only.

Restates the reference's allocator contract (``edgerag/cache/allocator.py:76-254``,
``tests/test_allocator.py``): a fresh pool hands out 0, 1, 2, ... and reuses the most recently
released block first; ``allocate`` is all or nothing; ``blocks_needed = ceil``; releasing a free
block raises; copy-on-write returns the block itself when private. A randomized run checks the
array-backed pool against a plain-Python model of the same contract.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from edgerag_amd.cache.allocator import (AllocatorError, BlockAllocator, DoubleFreeError,
                                         OutOfBlocksError)
from edgerag_amd.cache.block_table import BlockTable, pack_tables, step_slots


def test_hand_out_order_is_lifo_from_block_zero() -> None:
    a = BlockAllocator(8, 16)
    assert a.allocate(3) == [0, 1, 2]
    a.free([1])
    a.free([0])
    assert a.allocate(2) == [0, 1]  # most recently released first
    assert a.allocate(1) == [3]


def test_allocate_is_all_or_nothing() -> None:
    a = BlockAllocator(4, 16)
    a.allocate(3)
    with pytest.raises(OutOfBlocksError):
        a.allocate(2)
    assert a.num_free == 1 and a.counters.refusals == 1
    a.check_invariants()


def test_blocks_needed_is_ceil_division() -> None:
    a = BlockAllocator(4, 16)
    assert [a.blocks_needed(n) for n in (0, 1, 15, 16, 17, 32, 33)] == [0, 1, 1, 1, 2, 2, 3]
    with pytest.raises(ValueError):
        a.blocks_needed(-1)


def test_double_free_and_bad_ids_change_nothing() -> None:
    a = BlockAllocator(8, 16)
    blocks = a.allocate(2)
    with pytest.raises(DoubleFreeError):
        a.free([blocks[0], blocks[0]])  # one owner, two releases
    assert a.refcount(blocks[0]) == 1  # validated before any count moved
    with pytest.raises(AllocatorError):
        a.free([blocks[1], 99])
    assert a.refcount(blocks[1]) == 1
    with pytest.raises(AllocatorError):
        a.incref([5])  # free block
    a.check_invariants()


def test_sharing_and_copy_on_write() -> None:
    a = BlockAllocator(8, 16)
    (b,) = a.allocate(1)
    assert a.copy_on_write(b) == b  # private: written in place
    a.incref([b])
    assert a.is_shared(b)
    fresh = a.copy_on_write(b)
    assert fresh != b and a.refcount(b) == 1 and a.refcount(fresh) == 1
    assert a.free([b, fresh]) == 2
    a.check_invariants()


def test_free_with_repeated_ids_releases_each_ownership() -> None:
    a = BlockAllocator(8, 16)
    b, c = a.allocate(2)
    a.incref([b, b])
    assert a.free([b, c, b]) == 1  # c back; b drops to 1 owner
    assert a.refcount(b) == 1
    assert a.free([b]) == 1
    assert a.num_free == 8
    a.check_invariants()


def test_randomized_against_a_list_model() -> None:
    rng = random.Random(7)
    a = BlockAllocator(24, 4)
    refs = [0] * 24
    stack = list(range(23, -1, -1))
    owned: list[int] = []
    for _ in range(3000):
        op = rng.random()
        if op < 0.45:
            n = rng.randint(0, 6)
            if n > len(stack):
                with pytest.raises(OutOfBlocksError):
                    a.allocate(n)
                continue
            want = [stack.pop() for _ in range(n)]
            for b in want:
                refs[b] = 1
            assert a.allocate(n) == want
            owned += want
        elif op < 0.6 and owned:
            b = rng.choice(owned)
            refs[b] += 1
            owned.append(b)
            a.incref([b])
        elif op < 0.7 and owned:
            b = rng.choice(owned)
            if refs[b] == 1:
                assert a.copy_on_write(b) == b
            elif not stack:
                with pytest.raises(OutOfBlocksError):
                    a.copy_on_write(b)
            else:  # a private copy takes over one ownership
                fresh = stack.pop()
                refs[b] -= 1
                refs[fresh] = 1
                owned.remove(b)
                owned.append(fresh)
                assert a.copy_on_write(b) == fresh
        elif owned:
            picks = rng.sample(owned, min(len(owned), rng.randint(1, 3)))
            back = 0
            for b in picks:
                owned.remove(b)
                refs[b] -= 1
                if refs[b] == 0:
                    stack.append(b)
                    back += 1
            assert a.free(picks) == back
        assert a.num_free == len(stack)
        ids = np.arange(24)
        assert a.shared_count(ids) == sum(1 for r in refs if r > 1)
        a.check_invariants()


def test_table_growth_is_all_or_nothing_and_counts_blocks() -> None:
    a = BlockAllocator(4, 16)
    t = BlockTable(a)
    assert t.append(16) == [0] and t.num_blocks == 1  # exact multiple: no spare block
    assert t.append(1) == [1]
    other = BlockTable(a)
    other.append(32)
    with pytest.raises(OutOfBlocksError):
        t.append(40)
    assert t.num_tokens == 17 and t.num_blocks == 2  # unchanged
    assert t.locate(16) == (1, 0)
    with pytest.raises(IndexError):
        t.locate(17)  # never written
    assert t.shrink_to(10) == 1 and t.num_blocks == 1
    assert t.free() == 1 and a.num_free == 2


def test_slots_pack_and_step_helpers() -> None:
    a = BlockAllocator(16, 4)
    a.allocate(5)  # offset the ids
    t1, t2 = BlockTable(a), BlockTable(a)
    t1.append(6)
    t2.append(9)
    assert t1.slots(0, 6).tolist() == [20, 21, 22, 23, 24, 25]
    bt = pack_tables([t1, t2])
    assert bt.shape == (2, 3) and bt[0].tolist() == [5, 6, -1] and bt[1].tolist() == [7, 8, 9]
    assert step_slots([t1, t2], [1, 2]).tolist() == [25, 35, 36]
    fork = t2.fork()
    assert a.is_shared(7) and fork.unshare(2) == (9, 10)
    assert fork.blocks == [7, 8, 10] and t2.blocks == [7, 8, 9]


# --- the executor's step reservation ----------------------------------------------------------


def _executor(num_blocks, max_pos=512):
    from edgerag_amd.core.model import EdgeRagDecoder
    from edgerag_amd.core.spec import ModelSpec
    from edgerag_amd.serve.executor import ModelExecutor

    spec = ModelSpec("tiny", "llama", 1, 64, 2, 2, 32, 64, max_pos, 10000.0, pad_token_id=0,
                     intermediate_size=64)
    model = EdgeRagDecoder(spec, 8, None, "cpu", torch.float32)
    alloc = BlockAllocator(num_blocks, 16)
    return ModelExecutor(model, spec, alloc, "cpu", torch.float32, chunk_size=64), alloc


def test_a_step_that_does_not_fit_changes_nothing() -> None:
    """The second request of a batch cannot get its blocks: the executor refuses the whole step
    before reserving anything, so the first request's table is not advanced either."""
    from edgerag_amd.sched.request import Request
    from edgerag_amd.sched.scheduler import Batch
    from edgerag_amd.serve.executor import StepDoesNotFit

    ex, alloc = _executor(6)
    r1 = Request("a", list(range(1, 40)), max_new_tokens=2)  # 3 blocks
    r2 = Request("b", list(range(1, 70)), max_new_tokens=2)  # 4 blocks: 7 > 6
    for r in (r1, r2):
        r.move_to(r.state.__class__.PREFILLING)
    with pytest.raises(StepDoesNotFit) as err:
        ex.execute(Batch(0, prefill=[r1, r2]))
    assert err.value.blocks_needed == 3 + 4
    assert alloc.num_free == 6
    assert r1.cache.seq_len == 0 and r2.cache.seq_len == 0
    assert r1.cache.table.num_blocks == 0 and r2.cache.table.num_blocks == 0


def test_positions_past_the_rope_table_are_refused() -> None:
    from edgerag_amd.sched.request import Request
    from edgerag_amd.sched.scheduler import Batch

    ex, alloc = _executor(64, max_pos=100)
    r = Request("a", list(range(1, 120)), max_new_tokens=2)
    r.move_to(r.state.__class__.PREFILLING)
    r.prefill_offset = 64
    r.cache = ex._cache_for(r)
    r.cache.table.append(64)
    with pytest.raises(ValueError, match="past the model's 100 positions"):
        ex.execute(Batch(0, prefill=[r]))
    assert r.cache.seq_len == 64 and alloc.num_used == 4
    assert r.cache.table.blocks == [0, 1, 2, 3]
