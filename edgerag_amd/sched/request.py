"""A generation request and its lifecycle, as the scheduler and the packed executor see it.

The lifecycle is an explicit state machine; :meth:`Request.move_to` refuses transitions that are
not in :data:`TRANSITIONS`, so a bookkeeping bug surfaces where it happens instead of as a request
that decodes without KV or frees its blocks twice::

    WAITING --admit--> PREFILLING --last chunk--> DECODING --stop--> FINISHED
       ^  \\                 |                       |
       |   `-----------------+------ reject ---------+-----> REJECTED
       `---- preempt --------+-----------------------'
    SWAPPED (KV held in host memory) --readmit--> PREFILLING / DECODING

The prompt of a request is what the model still has to *read* before it can decode: the prompt
tokens, and after a recompute preemption also the tokens it had already generated (their KV was
dropped with the blocks). :attr:`prefill_len` counts both; :meth:`prefill_ids` slices them.
``prompt_embeds`` (``(1, prompt_len, hidden)``, optional) replaces the embedding lookup of the
prompt part, which is how retrieval-augmented prompts with visual tokens reach the decoder
(``edgerag/serve/executor.py:103-110`` in the reference).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from typing import Any


class RequestState(str, Enum):
    WAITING = "waiting"
    PREFILLING = "prefilling"
    DECODING = "decoding"
    SWAPPED = "swapped"
    FINISHED = "finished"
    REJECTED = "rejected"

    def __str__(self) -> str:
        return self.value


S = RequestState
#: Legal moves of the lifecycle.
TRANSITIONS: dict[RequestState, frozenset[RequestState]] = {
    S.WAITING: frozenset({S.PREFILLING, S.REJECTED}),
    S.PREFILLING: frozenset({S.DECODING, S.WAITING, S.SWAPPED, S.REJECTED}),
    S.DECODING: frozenset({S.FINISHED, S.WAITING, S.SWAPPED, S.REJECTED}),
    S.SWAPPED: frozenset({S.PREFILLING, S.DECODING, S.WAITING, S.REJECTED}),
    S.FINISHED: frozenset(),
    S.REJECTED: frozenset(),
}
#: States in which a request holds pool blocks (and so can be preempted).
HOLDS_BLOCKS = frozenset({S.PREFILLING, S.DECODING})


class TransitionError(RuntimeError):
    """A lifecycle move that the state machine does not allow."""


@dataclass(eq=False)
class Request:
    request_id: str
    prompt_token_ids: list[int]
    max_new_tokens: int = 64
    prompt_embeds: Any = None
    state: RequestState = RequestState.WAITING
    #: Tokens of :meth:`prefill_ids` already read into the KV cache.
    prefill_offset: int = 0
    generated_token_ids: list[int] = field(default_factory=list)
    #: The request's KV cache while it holds blocks (created by the executor).
    cache: Any = None
    #: Generated tokens folded back into the prompt by a recompute preemption.
    refeed: int = 0
    #: A swapped-out KV record while the request waits in host memory (set by the preemptor).
    swap: Any = None
    preemptions: int = 0
    reject_reason: str | None = None
    # Iteration stamps (scheduler steps) and optional clock stamps (load drivers).
    arrival_step: int = 0
    admitted_step: int | None = None
    first_token_step: int | None = None
    finished_step: int | None = None
    arrival_time: float | None = None
    first_token_time: float | None = None
    finish_time: float | None = None

    # --- sizes --------------------------------------------------------------------------------

    @property
    def prompt_len(self) -> int:
        return len(self.prompt_token_ids)

    @property
    def num_generated(self) -> int:
        return len(self.generated_token_ids)

    @property
    def total_tokens(self) -> int:
        """Positions the request occupies once every token so far is in the KV cache."""
        return self.prompt_len + self.num_generated

    @property
    def final_tokens(self) -> int:
        """Positions the request can ever occupy: prompt plus its whole generation budget."""
        return self.prompt_len + self.max_new_tokens

    @property
    def prefill_len(self) -> int:
        return self.prompt_len + self.refeed

    @property
    def prefill_done(self) -> bool:
        return self.prefill_offset >= self.prefill_len

    @property
    def is_terminal(self) -> bool:
        return not TRANSITIONS[self.state]

    def prefill_ids(self, start: int, end: int) -> list[int]:
        """Token ids of prefill positions ``[start, end)`` (prompt, then re-fed tokens)."""
        if not 0 <= start <= end <= self.prefill_len:
            raise IndexError(f"prefill slice [{start}, {end}) of {self.prefill_len} positions")
        head = self.prompt_token_ids[start : min(end, self.prompt_len)]
        if end <= self.prompt_len:
            return head
        lo = max(start, self.prompt_len) - self.prompt_len
        return head + self.generated_token_ids[lo : end - self.prompt_len]

    def next_prefill_chunk(self, chunk_size: int) -> list[int]:
        """The ids of the next slice to read, at most ``chunk_size`` (nothing is consumed)."""
        if chunk_size < 1:
            raise ValueError(f"chunk size must be >= 1, got {chunk_size}")
        return self.prefill_ids(self.prefill_offset,
                                min(self.prefill_len, self.prefill_offset + chunk_size))

    # --- lifecycle ----------------------------------------------------------------------------

    def move_to(self, state: RequestState) -> None:
        if state not in TRANSITIONS[self.state]:
            raise TransitionError(f"{self.request_id}: {self.state} -> {state} is not a legal move")
        self.state = state

    def advance_prefill(self, n_tokens: int) -> None:
        """Count ``n_tokens`` more prefill positions as read."""
        if n_tokens < 0 or self.prefill_offset + n_tokens > self.prefill_len:
            raise ValueError(
                f"{self.request_id}: reading {n_tokens} more positions from offset "
                f"{self.prefill_offset} overruns the {self.prefill_len} to prefill"
            )
        self.prefill_offset += n_tokens

    def append_token(self, token_id: int, step: int) -> None:
        if self.first_token_step is None:
            self.first_token_step = step
        self.generated_token_ids.append(int(token_id))

    def should_stop(self, eos_token_id: int | None = None) -> bool:
        """Budget exhausted, or the last token is the end-of-sequence id."""
        if self.num_generated >= self.max_new_tokens:
            return True
        return (eos_token_id is not None and self.num_generated > 0
                and self.generated_token_ids[-1] == eos_token_id)

    def requeue_for_recompute(self) -> None:
        """After a preemption that dropped the KV: read the prompt and every generated token
        again (the next token comes out of that prefill's last position)."""
        self.cache = None
        self.swap = None
        self.refeed = self.num_generated
        self.prefill_offset = 0
        if self.state is not RequestState.WAITING:
            self.move_to(RequestState.WAITING)

    def ttft_steps(self) -> int | None:
        return None if self.first_token_step is None else self.first_token_step - self.arrival_step

    def summary(self) -> dict[str, Any]:
        return {
            "id": self.request_id, "state": str(self.state),
            "tokens": {"prompt": self.prompt_len, "generated": self.num_generated,
                       "budget": self.max_new_tokens, "prefilled": self.prefill_offset},
            "steps": {"arrival": self.arrival_step, "admitted": self.admitted_step,
                      "first_token": self.first_token_step, "finished": self.finished_step},
            "preemptions": self.preemptions, "reject_reason": self.reject_reason,
        }
