"""Scheduler and request state machine (host-only), restating the reference's scheduler tests:
decode first, at most one prefill per step, admission budgeted on prompt + max_new against the
free pool minus the CoW reserve, FIFO blocking, pool conservation under a randomized soak
(``tests/test_scheduler.py`` in the reference, ``:291-316`` for the soak)."""

from __future__ import annotations

import random

import pytest

from edgerag_amd.cache.allocator import BlockAllocator
from edgerag_amd.cache.block_table import BlockTable
from edgerag_amd.sched.request import Request, RequestState
from edgerag_amd.sched.scheduler import Scheduler, SchedulerConfig
from edgerag_amd.serve.replay import poisson_arrivals, synthetic_requests


def _req(i: int, prompt: int = 40, new: int = 4) -> Request:
    return Request(request_id=f"r{i}", prompt_token_ids=list(range(1, prompt + 1)),
                   max_new_tokens=new)


class _FakeCache:
    """Holds real allocator blocks the way a paged cache does (grows per token)."""

    def __init__(self, allocator: BlockAllocator) -> None:
        self.table = BlockTable(allocator=allocator)

    def grow(self, n: int) -> None:
        self.table.append(n)

    def free(self) -> int:
        return self.table.free()


def _run_step(s: Scheduler, alloc: BlockAllocator, chunk: int, rng: random.Random | None = None):
    batch = s.schedule()
    for r in batch.prefill:
        if r.cache is None:
            r.cache = _FakeCache(alloc)
        n = min(chunk, r.prompt_len - r.prefill_offset)
        r.cache.grow(n)
        s.on_prefill_chunk(r, n)
        if r.prefill_done:
            s.on_token(r, 7)
    for r in batch.decode:
        r.cache.grow(1)
        tok = 2 if rng is not None and rng.random() < 0.05 else 7
        s.on_token(r, tok)
    s.end_step()
    return batch


def test_decode_first_and_one_prefill_per_step() -> None:
    alloc = BlockAllocator(256, 16)
    s = Scheduler(alloc, SchedulerConfig(max_batch_size=8))
    for i in range(4):
        s.add_request(_req(i, prompt=40, new=10))
    b0 = s.schedule()
    assert [r.request_id for r in b0.prefill] == ["r0"] and not b0.decode
    s.on_prefill_chunk(b0.prefill[0], 40)
    s.on_token(b0.prefill[0], 5)
    s.end_step()
    b1 = s.schedule()
    assert [r.request_id for r in b1.decode] == ["r0"]
    assert [r.request_id for r in b1.prefill] == ["r1"]


def test_chunked_prefill_progress_and_state_transitions() -> None:
    alloc = BlockAllocator(64, 16)
    s = Scheduler(alloc)
    r = _req(0, prompt=20, new=2)
    s.add_request(r)
    b = s.schedule()
    assert r.state is RequestState.PREFILLING and r.next_prefill_chunk(8) == r.prompt_token_ids[:8]
    s.on_prefill_chunk(r, 8)
    assert r.state is RequestState.PREFILLING and r.prefill_offset == 8
    s.on_prefill_chunk(r, 12)
    assert r.state is RequestState.DECODING
    with pytest.raises(ValueError):
        r.advance_prefill(1)
    s.on_token(r, 3)
    s.on_token(r, 4)
    assert r.state is RequestState.FINISHED and s.finished == [r] and b.size == 1


def test_admission_budgets_prompt_plus_generation_and_keeps_the_reserve() -> None:
    alloc = BlockAllocator(40, 16)
    alloc.allocate(20)  # held by someone else: 20 free, reserve 4 -> 16 admissible now
    s = Scheduler(alloc, SchedulerConfig(cow_reserve_blocks=4))
    big = _req(0, prompt=200, new=57)  # ceil(257/16) = 17 > 16: blocked
    s.add_request(big)
    s.add_request(_req(1, prompt=10, new=2))
    b = s.schedule()
    assert b.is_empty and s.counters.queue_held == 1  # FIFO: the small one waits behind
    assert s.blocks_required(big) == 17
    fits = _req(2, prompt=200, new=56)  # 16 blocks
    s2 = Scheduler(BlockAllocator(20, 16), SchedulerConfig(cow_reserve_blocks=4))
    s2.add_request(fits)
    assert s2.schedule().prefill == [fits]


def test_max_batch_size_caps_running_requests() -> None:
    alloc = BlockAllocator(1024, 16)
    s = Scheduler(alloc, SchedulerConfig(max_batch_size=3))
    for i in range(6):
        s.add_request(_req(i, prompt=8, new=50))
    for _ in range(6):
        _run_step(s, alloc, chunk=512)
    assert len(s.running) == 3 and len(s.waiting) == 3


def test_randomized_soak_conserves_the_pool() -> None:
    rng = random.Random(0)
    alloc = BlockAllocator(96, 16)
    s = Scheduler(alloc, SchedulerConfig(max_batch_size=5, eos_token_id=2))
    for i in range(40):
        s.add_request(_req(i, prompt=rng.randint(1, 200), new=rng.randint(1, 40)))
    for _ in range(5000):
        if not s.has_work:
            break
        _run_step(s, alloc, chunk=rng.choice([8, 64, 512]), rng=rng)
        alloc.check_invariants()
        held = sum(r.cache.table.num_blocks for r in s.running if r.cache is not None)
        assert held == alloc.num_used
    assert not s.has_work and len(s.finished) == 40
    assert alloc.num_free == alloc.num_blocks


def test_poisson_arrivals_and_trace_are_seeded_and_shaped() -> None:
    a, b = poisson_arrivals(64, 0.2, 5), poisson_arrivals(64, 0.2, 5)
    assert a == b and all(x < y for x, y in zip(a, a[1:]))
    assert 0.5 * 64 / 0.2 < a[-1] < 1.5 * 64 / 0.2
    reqs = synthetic_requests(256, 49152, 1)
    lens = sorted(r.prompt_len for r in reqs)
    assert lens[0] >= 256 and lens[-1] <= 7472
    assert 2400 < lens[len(lens) // 2] < 3600  # median 3000, lognormal sigma 0.6
    assert all(64 <= r.max_new_tokens <= 256 for r in reqs)
    with pytest.raises(ValueError):
        poisson_arrivals(3, 0.0, 1)


def test_illegal_lifecycle_moves_are_refused() -> None:
    from edgerag_amd.sched.request import TransitionError

    r = _req(0)
    with pytest.raises(TransitionError):
        r.move_to(RequestState.DECODING)  # WAITING -> DECODING skips prefill
    r.move_to(RequestState.PREFILLING)
    r.move_to(RequestState.DECODING)
    r.move_to(RequestState.FINISHED)
    assert r.is_terminal
    with pytest.raises(TransitionError):
        r.move_to(RequestState.WAITING)


def test_requests_that_can_never_fit_are_rejected_not_blocking() -> None:
    alloc = BlockAllocator(20, 16)
    s = Scheduler(alloc, SchedulerConfig(cow_reserve_blocks=4, max_model_len=300))
    too_long = _req(0, prompt=280, new=40)  # 320 positions > 300
    too_big = Request("r1", list(range(1, 200)), max_new_tokens=100)  # 19 blocks > 16 ever
    ok = _req(2, prompt=30, new=5)
    for r in (too_long, too_big, ok):
        s.add_request(r)
    b = s.schedule()
    assert b.prefill == [ok]
    assert too_long.state is RequestState.REJECTED and "positions" in too_long.reject_reason
    assert too_big.state is RequestState.REJECTED and s.rejected == [too_long, too_big]


def test_preempt_recompute_folds_generated_tokens_into_the_prefill() -> None:
    """Newest admission first; victims wait at the queue front in their old order; after a
    recompute preemption the request re-reads prompt + generated tokens, and its next token comes
    from that prefill's last position."""
    alloc = BlockAllocator(64, 16)
    s = Scheduler(alloc, SchedulerConfig(max_batch_size=4, max_prefills_per_step=4))
    reqs = [_req(i, prompt=20, new=8) for i in range(3)]
    for r in reqs:
        s.add_request(r)
    for _ in range(3):
        _run_step(s, alloc, chunk=512)
    assert all(r.state is RequestState.DECODING for r in reqs)
    held = [r.cache.table.num_blocks for r in reqs]
    need = alloc.num_free + held[2] + held[1]
    victims = s.preempt(need)
    assert victims == [reqs[1], reqs[2]] and list(s.waiting)[:2] == victims
    assert alloc.num_free == need and reqs[0].state is RequestState.DECODING
    v = reqs[2]
    gen = list(v.generated_token_ids)
    assert v.state is RequestState.WAITING and v.cache is None and v.preemptions == 1
    assert v.prefill_len == 20 + len(gen) and v.prefill_offset == 0
    assert v.prefill_ids(0, v.prefill_len) == v.prompt_token_ids + gen
    assert v.next_prefill_chunk(512) == v.prompt_token_ids + gen
    alloc.check_invariants()


def test_preempt_with_reject_policy_rejects_the_victims() -> None:
    from edgerag_amd.cache.preemption import PreemptionPolicy, Preemptor

    alloc = BlockAllocator(64, 16)
    s = Scheduler(alloc, SchedulerConfig(max_batch_size=4, max_prefills_per_step=4),
                  preemptor=Preemptor(alloc, PreemptionPolicy.REJECT))
    reqs = [_req(i, prompt=40, new=8) for i in range(2)]
    for r in reqs:
        s.add_request(r)
    _run_step(s, alloc, chunk=512)
    assert s.preempt(alloc.num_blocks) == []
    assert all(r.state is RequestState.REJECTED for r in reqs) and not s.running
    assert alloc.num_free == alloc.num_blocks
