"""Iteration-level continuous batching over the shared block pool (host only, no tensors).

Each call to :meth:`Scheduler.schedule` decides one iteration of the packed executor:

1. **Running work first.** Every running request that has finished its prefill decodes one token;
   prefilling requests contribute one chunk each, at most ``max_prefills_per_step`` of them.
2. **Admission**, in arrival order, while the batch has room (``max_batch_size`` running,
   ``max_prefills_per_step`` prefilling). A request is admitted only if its *final* size -- prompt
   plus its whole generation budget, ``blocks_needed(prompt + max_new)`` -- fits the free pool
   minus ``cow_reserve_blocks`` (the reference's rule, ``edgerag/sched/scheduler.py:120-176``):
   an admitted request then never needs a preemption to finish. The first request that does not
   fit holds the queue (no overtaking), unless it can *never* fit (larger than the pool, or past
   ``max_model_len`` positions): that one is rejected at once rather than blocking forever.
3. **Pressure relief.** :meth:`preempt` frees blocks by evicting running requests newest first;
   victims go back to the front of the queue. With a swap preemptor the victim's KV waits in host
   memory and is restored on readmission (no recompute); otherwise the request re-reads its
   prompt and generated tokens.

Bookkeeping calls (:meth:`on_prefill_chunk`, :meth:`on_token`, :meth:`end_step`) apply an
executor's :class:`~edgerag_amd.serve.executor.StepOutput`; every state change goes through the
request's state machine.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from typing import Any

from edgerag_amd.cache.allocator import BlockAllocator, OutOfBlocksError
from edgerag_amd.sched.request import HOLDS_BLOCKS, Request, RequestState

DEFAULT_PREFILL_CHUNK = 512


@dataclass
class SchedulerConfig:
    max_batch_size: int = 8
    prefill_chunk_size: int = DEFAULT_PREFILL_CHUNK
    cow_reserve_blocks: int = 4
    max_prefills_per_step: int = 1
    eos_token_id: int | None = None
    #: Largest number of positions a request may reach (the model's RoPE table); None: no bound.
    max_model_len: int | None = None


@dataclass
class Batch:
    """One iteration's work: requests that read a prefill chunk, requests that decode a token."""

    step: int
    prefill: list[Request] = field(default_factory=list)
    decode: list[Request] = field(default_factory=list)

    @property
    def is_empty(self) -> bool:
        return not (self.prefill or self.decode)

    @property
    def size(self) -> int:
        return len(self.prefill) + len(self.decode)

    @property
    def requests(self) -> list[Request]:
        return self.prefill + self.decode


@dataclass
class SchedulerCounters:
    iterations: int = 0
    admitted: int = 0
    finished: int = 0
    rejected: int = 0
    preempted: int = 0
    restored: int = 0
    chunks: int = 0
    tokens: int = 0
    queue_held: int = 0


class Scheduler:
    def __init__(self, allocator: BlockAllocator, config: SchedulerConfig | None = None,
                 preemptor: Any = None) -> None:
        """``preemptor``: a :class:`~edgerag_amd.cache.preemption.Preemptor` used by
        :meth:`preempt` (None: victims drop their KV and recompute)."""
        self.allocator = allocator
        self.config = config or SchedulerConfig()
        self.preemptor = preemptor
        self.waiting: deque[Request] = deque()
        self.running: list[Request] = []
        self.finished: list[Request] = []
        self.rejected: list[Request] = []
        self.step_index = 0
        self.counters = SchedulerCounters()

    # --- queue --------------------------------------------------------------------------------

    def add_request(self, request: Request) -> None:
        if request.state is not RequestState.WAITING:
            raise ValueError(f"{request.request_id} is {request.state}, not a new request")
        request.arrival_step = self.step_index
        self.waiting.append(request)

    @property
    def has_work(self) -> bool:
        return bool(self.waiting) or bool(self.running)

    @property
    def available_blocks(self) -> int:
        """Free blocks an admission may claim: the pool's free count minus the CoW reserve."""
        return max(0, self.allocator.num_free - self.config.cow_reserve_blocks)

    def blocks_required(self, request: Request) -> int:
        return self.allocator.blocks_needed(request.final_tokens)

    def _never_fits(self, request: Request) -> str | None:
        cap = self.config.max_model_len
        if cap is not None and request.final_tokens > cap:
            return (f"prompt {request.prompt_len} + budget {request.max_new_tokens} tokens exceed "
                    f"the model's {cap} positions")
        if self.blocks_required(request) > self.allocator.num_blocks - self.config.cow_reserve_blocks:
            return (f"needs {self.blocks_required(request)} blocks, the pool can ever offer "
                    f"{self.allocator.num_blocks - self.config.cow_reserve_blocks}")
        return None

    # --- the decision -------------------------------------------------------------------------

    def schedule(self) -> Batch:
        cfg = self.config
        batch = Batch(step=self.step_index)
        for request in self.running:
            if request.state is RequestState.DECODING:
                batch.decode.append(request)
            elif len(batch.prefill) < cfg.max_prefills_per_step:
                batch.prefill.append(request)
        while self.waiting and len(self.running) < cfg.max_batch_size:
            head = self.waiting[0]
            prefill_full = len(batch.prefill) >= cfg.max_prefills_per_step
            if prefill_full and not (head.swap is not None and head.prefill_done):
                break  # only a swapped-out decode can still join this iteration
            reason = self._never_fits(head)
            if reason is not None:
                self.waiting.popleft()
                self.reject(head, reason)
                continue
            if self.blocks_required(head) > self.available_blocks:
                self.counters.queue_held += 1
                break
            if not self._admit(head, batch, prefill_full):
                break
        return batch

    def _admit(self, request: Request, batch: Batch, prefill_full: bool) -> bool:
        """Move the queue head into the batch. A swapped-out request gets its KV back and resumes
        where it stopped; if the pool cannot take the KV back, it recomputes instead (and waits
        when this iteration has no prefill slot left). False: the head stays queued."""
        if request.swap is not None:
            try:
                self.preemptor.restore(request)
                self.counters.restored += 1
            except OutOfBlocksError:
                self.preemptor.discard(request)
                request.requeue_for_recompute()
                if prefill_full:
                    return False
        self.waiting.popleft()
        if request.admitted_step is None:
            request.admitted_step = self.step_index
        decoding = request.prefill_done
        request.move_to(RequestState.DECODING if decoding else RequestState.PREFILLING)
        self.running.append(request)
        self.counters.admitted += 1
        (batch.decode if decoding else batch.prefill).append(request)
        return True

    # --- progress -----------------------------------------------------------------------------

    def on_prefill_chunk(self, request: Request, n_tokens: int) -> None:
        request.advance_prefill(n_tokens)
        self.counters.chunks += 1
        if request.prefill_done:
            request.move_to(RequestState.DECODING)

    def on_token(self, request: Request, token_id: int) -> None:
        request.append_token(token_id, self.step_index)
        self.counters.tokens += 1
        if request.should_stop(self.config.eos_token_id):
            self.finish(request)

    def finish(self, request: Request) -> None:
        request.move_to(RequestState.FINISHED)
        request.finished_step = self.step_index
        self._drop_cache(request)
        self.running.remove(request)
        self.finished.append(request)
        self.counters.finished += 1

    def reject(self, request: Request, reason: str = "") -> None:
        """Refuse a request for good (waiting or running); its blocks return to the pool."""
        if request in self.waiting:
            self.waiting.remove(request)
        if request in self.running:
            self.running.remove(request)
        if request.swap is not None and self.preemptor is not None:
            self.preemptor.discard(request)
            request.swap = None
        self._drop_cache(request)
        request.reject_reason = reason or "rejected"
        request.finished_step = self.step_index
        request.move_to(RequestState.REJECTED)
        self.rejected.append(request)
        self.counters.rejected += 1

    def end_step(self) -> None:
        self.step_index += 1
        self.counters.iterations += 1

    @staticmethod
    def _drop_cache(request: Request) -> None:
        if request.cache is not None:
            request.cache.free()
            request.cache = None

    # --- pressure -----------------------------------------------------------------------------

    def preempt(self, blocks_needed: int) -> list[Request]:
        """Evict running requests, newest admission first, until ``blocks_needed`` blocks are
        free (or nothing is left to evict). Victims wait at the front of the queue in their
        original order. Returns them, oldest first."""
        victims: list[Request] = []
        for request in reversed(list(self.running)):
            if self.allocator.num_free >= blocks_needed:
                break
            if request.state not in HOLDS_BLOCKS:
                continue
            if self._evict(request):
                victims.append(request)
        victims.reverse()
        self.waiting.extendleft(reversed(victims))
        return victims

    def _evict(self, request: Request) -> bool:
        """Take a running request's blocks away. False when the preemptor's policy rejects it."""
        self.counters.preempted += 1
        request.preemptions += 1
        action = self.preemptor.evict(request) if self.preemptor is not None else "recompute"
        if action == "reject":
            self.reject(request, "preempted under memory pressure")
            return False
        self.running.remove(request)
        if action == "swap":  # the KV waits in host memory; progress is kept
            request.move_to(RequestState.SWAPPED)
        else:
            self._drop_cache(request)
            request.requeue_for_recompute()
        return True

    def snapshot(self) -> dict[str, Any]:
        c = self.counters
        return {
            "queue": {"waiting": len(self.waiting), "running": len(self.running),
                      "finished": len(self.finished), "rejected": len(self.rejected)},
            "events": {"iterations": c.iterations, "admitted": c.admitted,
                       "finished": c.finished, "rejected": c.rejected, "preempted": c.preempted,
                       "restored": c.restored, "prefill_chunks": c.chunks, "tokens": c.tokens,
                       "queue_held": c.queue_held},
        }
