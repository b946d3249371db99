"""Continuous-batching scheduler: iteration-level admission with chunked prefill (host-only).

Restates the policy of ``edgerag/sched/scheduler.py:41-202``, which is pure decision-making with
no tensors:

* decode first -- every running request past prefill decodes this iteration (``:150-158``);
* at most ``max_prefills_per_step`` prefilling requests per iteration (``:155-158``, ``:166-168``);
* admission in arrival order while ``len(running) < max_batch_size``, reserving the request's
  whole prompt plus generation budget (``blocks_needed(prompt + max_new)``) against the free pool
  minus ``cow_reserve_blocks`` (``:120-136``, ``:160-176``); the first request that does not fit
  blocks the queue (FIFO, no skipping).

Preemption (``:210-257``) is not wired into the reference executor and is not built here.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from typing import Any

from edgerag_amd.cache.allocator import BlockAllocator
from edgerag_amd.sched.request import Request, RequestState

DEFAULT_PREFILL_CHUNK = 512


@dataclass
class SchedulerConfig:
    """``scheduler.py:41-49``."""

    max_batch_size: int = 8
    prefill_chunk_size: int = DEFAULT_PREFILL_CHUNK
    cow_reserve_blocks: int = 4
    max_prefills_per_step: int = 1
    eos_token_id: int | None = None


@dataclass
class SchedulerStats:
    steps: int = 0
    admitted: int = 0
    finished: int = 0
    rejected: int = 0
    preempted: int = 0
    prefill_chunks: int = 0
    decode_steps: int = 0
    admission_blocked: int = 0
    extra: dict[str, Any] = field(default_factory=dict)


@dataclass
class Batch:
    """What runs this iteration (``scheduler.py:66-92``)."""

    step: int
    prefill: list[Request] = field(default_factory=list)
    decode: list[Request] = field(default_factory=list)

    @property
    def is_empty(self) -> bool:
        return not self.prefill and not self.decode

    @property
    def size(self) -> int:
        return len(self.prefill) + len(self.decode)

    @property
    def requests(self) -> list[Request]:
        return [*self.prefill, *self.decode]


class Scheduler:
    """Iteration-level scheduler over a shared block pool (``scheduler.py:95-202``)."""

    def __init__(self, allocator: BlockAllocator, config: SchedulerConfig | None = None) -> None:
        self.allocator = allocator
        self.config = config or SchedulerConfig()
        self.waiting: deque[Request] = deque()
        self.running: list[Request] = []
        self.finished: list[Request] = []
        self.step_index = 0
        self.stats = SchedulerStats()

    def add_request(self, request: Request) -> None:
        request.arrival_step = self.step_index
        request.state = RequestState.WAITING
        self.waiting.append(request)

    @property
    def has_work(self) -> bool:
        return bool(self.waiting or self.running)

    @property
    def available_blocks(self) -> int:
        """Blocks a new admission may use, after holding back the copy-on-write reserve."""
        return max(0, self.allocator.num_free - self.config.cow_reserve_blocks)

    def blocks_required(self, request: Request) -> int:
        """The request's final size: whole prompt plus every token it may generate."""
        return self.allocator.blocks_needed(request.prompt_len + request.max_new_tokens)

    def schedule(self) -> Batch:
        batch = Batch(step=self.step_index)
        for request in self.running:
            if request.state is RequestState.DECODING:
                batch.decode.append(request)
            elif (
                request.state is RequestState.PREFILLING
                and len(batch.prefill) < self.config.max_prefills_per_step
            ):
                batch.prefill.append(request)
        while (
            self.waiting
            and len(self.running) < self.config.max_batch_size
            and len(batch.prefill) < self.config.max_prefills_per_step
        ):
            request = self.waiting[0]
            if self.blocks_required(request) > self.available_blocks:
                self.stats.admission_blocked += 1
                break
            self.waiting.popleft()
            request.state = RequestState.PREFILLING
            request.admitted_step = self.step_index
            self.running.append(request)
            self.stats.admitted += 1
            batch.prefill.append(request)
        return batch

    def on_prefill_chunk(self, request: Request, n_tokens: int) -> None:
        request.advance_prefill(n_tokens)
        self.stats.prefill_chunks += 1
        if request.prefill_done:
            request.state = RequestState.DECODING

    def on_token(self, request: Request, token_id: int) -> None:
        request.append_token(token_id, self.step_index)
        self.stats.decode_steps += 1
        if request.should_stop(self.config.eos_token_id):
            self.finish(request)

    def finish(self, request: Request) -> None:
        request.state = RequestState.FINISHED
        request.finished_step = self.step_index
        if request.cache is not None:
            request.cache.free()
            request.cache = None
        if request in self.running:
            self.running.remove(request)
        self.finished.append(request)
        self.stats.finished += 1

    def end_step(self) -> None:
        self.step_index += 1
        self.stats.steps += 1
