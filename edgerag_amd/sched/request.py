"""Request lifecycle for continuous batching (host-only, no tensors).

Restates ``edgerag/sched/request.py:19-172``. The states, the chunked-prefill cursor
``prefill_offset`` and the stop rule are the reference's own. ``StrEnum`` (Python 3.11) is written
as ``str, Enum``, which compares and prints the same.
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


PREEMPTABLE = (RequestState.PREFILLING, RequestState.DECODING)
TERMINAL = (RequestState.FINISHED, RequestState.REJECTED)


@dataclass
class Request:
    """One in-flight generation request (``request.py:40-172``)."""

    request_id: str
    prompt_token_ids: list[int]
    max_new_tokens: int = 64
    arrival_step: int = 0
    state: RequestState = RequestState.WAITING
    prefill_offset: int = 0
    generated_token_ids: list[int] = field(default_factory=list)
    cache: Any = None
    prompt_embeds: Any = None
    admitted_step: int | None = None
    first_token_step: int | None = None
    finished_step: int | None = None
    preemptions: int = 0
    #: Wall-clock (or virtual-clock) stamps a load driver may fill in; unused by the scheduler.
    arrival_time: float | None = None
    first_token_time: float | None = None
    finish_time: float | None = None

    @property
    def prompt_len(self) -> int:
        return len(self.prompt_token_ids)

    @property
    def prefill_done(self) -> bool:
        return self.prefill_offset >= self.prompt_len

    @property
    def num_generated(self) -> int:
        return len(self.generated_token_ids)

    @property
    def total_tokens(self) -> int:
        """Positions the request occupies in the KV cache: prompt plus generated tokens."""
        return self.prompt_len + self.num_generated

    @property
    def is_terminal(self) -> bool:
        return self.state in TERMINAL

    def next_prefill_chunk(self, chunk_size: int) -> list[int]:
        """The next prompt slice, without advancing (``request.py:98-107``)."""
        if chunk_size <= 0:
            raise ValueError(f"chunk_size must be positive, got {chunk_size}")
        end = min(self.prefill_offset + chunk_size, self.prompt_len)
        return self.prompt_token_ids[self.prefill_offset : end]

    def advance_prefill(self, n_tokens: int) -> None:
        if n_tokens < 0:
            raise ValueError(f"cannot advance prefill by {n_tokens}")
        if self.prefill_offset + n_tokens > self.prompt_len:
            raise ValueError(
                f"{self.request_id}: prefill would advance to {self.prefill_offset + n_tokens} "
                f"past prompt length {self.prompt_len}"
            )
        self.prefill_offset += n_tokens

    def append_token(self, token_id: int, step: int) -> None:
        if self.first_token_step is None:
            self.first_token_step = step
        self.generated_token_ids.append(token_id)

    def should_stop(self, eos_token_id: int | None = None) -> bool:
        if self.num_generated >= self.max_new_tokens:
            return True
        return bool(
            eos_token_id is not None
            and self.generated_token_ids
            and self.generated_token_ids[-1] == eos_token_id
        )

    def mark_preempted(self) -> None:
        self.state = RequestState.SWAPPED
        self.preemptions += 1

    def reset_for_recompute(self) -> None:
        self.prefill_offset = 0
        self.cache = None
        self.state = RequestState.WAITING

    def ttft_steps(self) -> int | None:
        if self.first_token_step is None:
            return None
        return self.first_token_step - self.arrival_step

    def to_dict(self) -> dict[str, Any]:
        return {
            "request_id": self.request_id,
            "state": self.state.value,
            "prompt_len": self.prompt_len,
            "prefill_offset": self.prefill_offset,
            "generated": self.num_generated,
            "total_tokens": self.total_tokens,
            "preemptions": self.preemptions,
            "ttft_steps": self.ttft_steps(),
            "arrival_step": self.arrival_step,
            "finished_step": self.finished_step,
        }
