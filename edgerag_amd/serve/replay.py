"""Serving-load driver for BASELINE config 5: a seeded Poisson request trace replayed through the
scheduler and the ragged executor.

* :func:`poisson_arrivals` restates ``bench/load.py:134-149``: cumulative exponential gaps from
  ``random.Random(seed).expovariate(rate)``, fixed up front by ``(n, rate, seed)``.
* :func:`synthetic_requests`: prompts of random token ids with lognormal lengths (median 3000,
  sigma 0.6) clamped to [256, 7472], and 64-256 greedy output tokens (no EOS), seeded.
* :func:`replay` runs the engine loop (``serve/engine.py:169-214``) against the arrival schedule
  and reports the reference's metric, output tokens per second = generated tokens / (last finish
  - first arrival) (``bench/load.py:110-131``).

The clock: ``"virtual"`` advances by the measured wall time of each iteration and jumps over idle
gaps to the next arrival, so a 64-request trace at 12 req/min (320 s of arrivals) replays in the
time the GPU is actually busy, with the same admission order and the same per-request timestamps
a real-time replay would see when every iteration takes what it took. ``"saturated"`` submits
every request at t = 0: the capacity figure.
"""

from __future__ import annotations

import math
import random
import time
from dataclasses import dataclass, field

import numpy as np
import torch

from edgerag_amd.sched.request import Request
from edgerag_amd.sched.scheduler import Scheduler
from edgerag_amd.serve.executor import ModelExecutor, apply_output


def poisson_arrivals(n: int, rate_hz: float, seed: int) -> list[float]:
    if rate_hz <= 0:
        raise ValueError(f"arrival rate must be positive, got {rate_hz}")
    rng = random.Random(seed)
    offsets, clock = [], 0.0
    for _ in range(n):
        clock += rng.expovariate(rate_hz)
        offsets.append(clock)
    return offsets


def synthetic_requests(n: int, vocab_size: int, seed: int, median: float = 3000.0,
                       sigma: float = 0.6, min_len: int = 256, max_len: int = 7472,
                       min_new: int = 64, max_new: int = 256) -> list[Request]:
    rng = np.random.default_rng(seed)
    lens = np.clip(np.round(np.exp(np.log(median) + sigma * rng.standard_normal(n))),
                   min_len, max_len).astype(int)
    outs = rng.integers(min_new, max_new + 1, size=n)
    reqs = []
    for i in range(n):
        ids = rng.integers(1, vocab_size - 1, size=int(lens[i])).tolist()
        reqs.append(Request(request_id=f"req{i:03d}", prompt_token_ids=ids,
                            max_new_tokens=int(outs[i])))
    return reqs


@dataclass
class ReplayResult:
    mode: str
    n_requests: int
    n_finished: int
    generated_tokens: int
    prompt_tokens: int
    window_s: float
    busy_s: float
    steps: int
    step_ms: list[float] = field(default_factory=list)
    ttft_s: list[float] = field(default_factory=list)

    @property
    def output_tokens_per_s(self) -> float:
        return self.generated_tokens / self.window_s if self.window_s > 0 else 0.0

    def summary(self) -> dict:
        steps = np.asarray(self.step_ms) if self.step_ms else np.zeros(1)
        ttft = np.asarray(self.ttft_s) if self.ttft_s else np.zeros(1)
        return {
            "mode": self.mode,
            "output_tok_per_s": round(self.output_tokens_per_s, 2),
            "n_requests": self.n_requests,
            "n_finished": self.n_finished,
            "generated_tokens": self.generated_tokens,
            "prompt_tokens": self.prompt_tokens,
            "window_s": round(self.window_s, 3),
            "gpu_busy_s": round(self.busy_s, 3),
            "iterations": self.steps,
            "iteration_ms_p50": round(float(np.percentile(steps, 50)), 3),
            "iteration_ms_p99": round(float(np.percentile(steps, 99)), 3),
            "ttft_s_p50": round(float(np.percentile(ttft, 50)), 3),
            "ttft_s_p99": round(float(np.percentile(ttft, 99)), 3),
        }


def replay(scheduler: Scheduler, executor: ModelExecutor, requests: list[Request],
           arrivals: list[float] | None, mode: str = "virtual",
           max_steps: int = 1_000_000) -> ReplayResult:
    """Run ``requests`` (arriving at ``arrivals`` seconds; all at 0 when None) to completion."""
    order = sorted(range(len(requests)), key=lambda i: arrivals[i] if arrivals else 0.0)
    at = [arrivals[i] if arrivals else 0.0 for i in order]
    pending = [requests[i] for i in order]
    nxt, now, busy, steps = 0, 0.0, 0.0, 0
    step_ms: list[float] = []
    sync = executor.device.type == "cuda"
    while steps < max_steps:
        while nxt < len(pending) and at[nxt] <= now:
            req = pending[nxt]
            req.arrival_time = at[nxt]
            scheduler.add_request(req)
            nxt += 1
        if not scheduler.has_work:
            if nxt >= len(pending):
                break
            now = at[nxt]  # idle until the next arrival
            continue
        batch = scheduler.schedule()
        if batch.is_empty:
            raise RuntimeError("scheduler has work but scheduled nothing (pool too small?)")
        t0 = time.perf_counter()
        output = executor.execute(batch)
        if sync:
            torch.cuda.synchronize(executor.device)
        dt = time.perf_counter() - t0
        now += dt
        busy += dt
        steps += 1
        step_ms.append(dt * 1e3)
        apply_output(scheduler, batch, output)
        for request in batch.requests:
            if request.first_token_time is None and request.generated_token_ids:
                request.first_token_time = now
            if request.is_terminal and request.finish_time is None:
                request.finish_time = now
    done = [r for r in requests if r.finish_time is not None]
    first = min((r.arrival_time for r in requests if r.arrival_time is not None), default=0.0)
    last = max((r.finish_time for r in done), default=first)
    return ReplayResult(
        mode=mode, n_requests=len(requests), n_finished=len(done),
        generated_tokens=sum(r.num_generated for r in requests),
        prompt_tokens=sum(r.prompt_len for r in requests), window_s=last - first, busy_s=busy,
        steps=steps, step_ms=step_ms,
        ttft_s=[r.first_token_time - r.arrival_time for r in done
                if r.first_token_time is not None],
    )
