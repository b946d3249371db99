"""The batch executor: one packed ragged forward per scheduler iteration.

Contract of the reference ``ModelExecutor`` (``edgerag/serve/executor.py:57-156``):
``execute(batch) -> StepOutput``, where each prefilling request advances by at most
``chunk_size`` prompt tokens (``:116-130``), the final prefill chunk emits the request's first
generated token (``:131-136``), each decoding request feeds its last generated token and emits the
next (``:138-154``), and one KV arena is allocated once and shared by every request's block
table (``:76-83``, B-05). Greedy selection is ``argmax`` over the last position's logits.

What changes: the reference runs one decoder forward per request per iteration, each with its own
host-to-device index uploads and a device-to-host argmax. Here the whole batch is one forward:
the host builds the step's metadata (token ids, logical positions, pool slots, cu_seqlens,
context lengths, block tables, the attention work plan, the rows whose logits are read) and
uploads it in one pinned copy; the argmax of every emitting request comes back in one copy.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

from edgerag_amd import kernels
from edgerag_amd.cache.allocator import BlockAllocator
from edgerag_amd.cache.paged import PagedKVCache
from edgerag_amd.core.model import EdgeRagDecoder, StepInputs
from edgerag_amd.core.spec import ModelSpec
from edgerag_amd.sched.request import Request
from edgerag_amd.sched.scheduler import Batch

DEFAULT_CHUNK_SIZE = 512


@dataclass
class StepOutput:
    """``edgerag/serve/engine.py:59-71``: tokens emitted and prompt tokens consumed, by request."""

    tokens: dict[str, int] = field(default_factory=dict)
    prefilled: dict[str, int] = field(default_factory=dict)


class ModelExecutor:
    def __init__(
        self,
        decoder: EdgeRagDecoder,
        spec: ModelSpec,
        allocator: BlockAllocator,
        device: torch.device,
        dtype: torch.dtype = torch.float16,
        chunk_size: int = DEFAULT_CHUNK_SIZE,
        decode_graphs: bool = True,
        max_decode_batch: int = 8,
    ) -> None:
        """``decode_graphs``: replay decode-only iterations (up to ``max_decode_batch`` requests)
        from HIP graphs captured per batch size; iterations with a prefill chunk run eagerly."""
        if chunk_size <= 0:
            raise ValueError(f"chunk_size must be positive, got {chunk_size}")
        self.decoder = decoder
        self.spec = spec
        self.allocator = allocator
        self.device = torch.device(device)
        self.dtype = dtype
        self.chunk_size = chunk_size
        shape = (spec.n_kv_heads, allocator.num_blocks, allocator.block_size, spec.head_dim)
        self.key_pool = [torch.zeros(shape, dtype=dtype, device=self.device)
                         for _ in range(spec.n_layers)]
        self.value_pool = [torch.zeros(shape, dtype=dtype, device=self.device)
                           for _ in range(spec.n_layers)]
        #: Logits of the last step's emitting rows (kept for inspection; no copy is made).
        self.last_logits: torch.Tensor | None = None
        self.decode_graphs = decode_graphs and self.device.type == "cuda"
        self.max_decode_batch = max_decode_batch
        self._fixed: kernels.FixedAttention | None = None
        self._graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor, torch.Tensor]] = {}
        self.graph_steps = 0

    @property
    def pool_bytes(self) -> int:
        per_tensor = self.key_pool[0].numel() * self.key_pool[0].element_size()
        return per_tensor * len(self.key_pool) * 2

    def _cache_for(self, request: Request) -> PagedKVCache:
        if request.cache is None:
            request.cache = PagedKVCache(self.spec, self.allocator, self.device, self.dtype,
                                         pool=self.key_pool, value_pool=self.value_pool)
        return request.cache

    @torch.inference_mode()
    def execute(self, batch: Batch) -> StepOutput:
        output = StepOutput()
        # (request, new tokens, emits a token, is a prefill chunk)
        entries: list[tuple[Request, list[int], bool, bool]] = []
        for request in batch.prefill:
            start = request.prefill_offset
            end = min(start + self.chunk_size, request.prompt_len)
            if end - start <= 0:
                continue
            entries.append((request, request.prompt_token_ids[start:end],
                            end >= request.prompt_len, True))
        for request in batch.decode:
            if not request.generated_token_ids:
                raise RuntimeError(
                    f"{request.request_id} reached decode with no generated token: prefill "
                    "completed without emitting one"
                )
            entries.append((request, [request.generated_token_ids[-1]], True, False))
        if not entries:
            return output

        qsl, ctx, ids, pos, slots, tables, rows, emitting = [0], [], [], [], [], [], [], []
        for request, toks, emits, _ in entries:
            cache = self._cache_for(request)
            n = len(toks)
            slots.append(cache.reserve(n))
            L = cache.seq_len
            ctx.append(L)
            pos.append(np.arange(L - n, L, dtype=np.int32))
            ids.extend(toks)
            qsl.append(qsl[-1] + n)
            tables.append(cache.table.blocks)
            if emits:
                rows.append(qsl[-1] - 1)
                emitting.append(request)
        bt = np.full((len(entries), max(len(t) for t in tables)), -1, np.int32)
        for r, t in enumerate(tables):
            bt[r, : len(t)] = t
        spec = self.spec
        extras = [np.concatenate(slots).astype(np.int32), np.concatenate(pos),
                  np.asarray(ids, np.int32), np.asarray(rows, np.int32)]
        if (self.decode_graphs and not batch.prefill and len(entries) <= self.max_decode_batch
                and self._stage_fixed(qsl, ctx, bt, extras)):
            logits, choice = self._replay_decode(len(entries))
            self.last_logits = logits
            tokens = choice.cpu().tolist()
            for request, token in zip(emitting, tokens):
                output.tokens[request.request_id] = int(token)
            self.graph_steps += 1
            return output
        plan, (slot_d, pos_d, ids_d, rows_d) = kernels.plan_attention(
            np.asarray(qsl, np.int32), np.asarray(ctx, np.int32), bt, spec.n_q_heads,
            spec.n_kv_heads, spec.head_dim, self.allocator.block_size, self.dtype, self.device,
            extras,
        )
        step = StepInputs(ids_d, pos_d, slot_d, rows_d, plan)
        if emitting:
            logits = self.decoder.logits(step, self.key_pool, self.value_pool)
            self.last_logits = logits
            tokens = kernels.argmax_rows(logits).cpu().tolist()
            for request, token in zip(emitting, tokens):
                output.tokens[request.request_id] = int(token)
        else:
            self.decoder.forward_hidden(step, self.key_pool, self.value_pool)
        for request, toks, _, is_prefill in entries:
            if is_prefill:
                output.prefilled[request.request_id] = len(toks)
        return output

    # --- decode iterations replayed from HIP graphs ------------------------------------------

    def _stage_fixed(self, qsl, ctx, bt, extras) -> bool:
        if self._fixed is None:
            spec = self.spec
            max_blocks = -(-spec.max_position_embeddings // self.allocator.block_size)
            cap = self.max_decode_batch
            self._fixed = kernels.FixedAttention(
                self.device, spec.n_q_heads, spec.n_kv_heads, spec.head_dim,
                self.allocator.block_size, self.dtype, cap, max_blocks, [cap, cap, cap, cap])
        return self._fixed.update(np.asarray(qsl, np.int32), np.asarray(ctx, np.int32), bt,
                                  extras)

    def _replay_decode(self, n: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Logits ``(n, vocab)`` of a staged decode-only step of ``n`` requests and their greedy
        tokens (int32 ``(n,)``), both computed inside the replayed graph."""
        entry = self._graphs.get(n)
        if entry is None:
            fx = self._fixed
            slots, pos, ids, rows = (e[:n] for e in fx.extras)
            step = StepInputs(ids, pos, slots, rows, fx)
            stream = torch.cuda.Stream(self.device)
            stream.wait_stream(torch.cuda.current_stream(self.device))
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(stream):
                # The staged metadata is already valid, so run once eagerly first (lets torch and
                # hipBLASLt settle their workspaces outside the capture); it computes this step's
                # logits, which the replay below recomputes identically.
                self.decoder.logits(step, self.key_pool, self.value_pool)
                with torch.cuda.graph(graph, stream=stream):
                    logits = self.decoder.logits(step, self.key_pool, self.value_pool)
                    choice = kernels.argmax_rows(logits)
            torch.cuda.current_stream(self.device).wait_stream(stream)
            entry = self._graphs[n] = (graph, logits, choice)
        graph, logits, choice = entry
        graph.replay()
        return logits, choice

    def to_dict(self) -> dict[str, Any]:
        return {
            "chunk_size": self.chunk_size,
            "pool_blocks": self.allocator.num_blocks,
            "block_size": self.allocator.block_size,
            "pool_bytes": self.pool_bytes,
            "dtype": str(self.dtype).replace("torch.", ""),
        }


def drive(scheduler, executor: ModelExecutor, max_steps: int = 100000, on_step=None) -> int:
    """The engine's scheduler/executor loop without threads (``tests/test_executor.py:54-70``,
    ``serve/engine.py:169-214``). Returns the number of iterations run."""
    steps = 0
    while scheduler.has_work and steps < max_steps:
        batch = scheduler.schedule()
        if batch.is_empty:
            break
        output = executor.execute(batch)
        apply_output(scheduler, batch, output)
        steps += 1
        if on_step is not None:
            on_step(batch, output)
    return steps


def apply_output(scheduler, batch: Batch, output: StepOutput) -> None:
    """``serve/engine.py:191-214``: advance prefill, append tokens, let the scheduler finish."""
    for request in batch.requests:
        consumed = output.prefilled.get(request.request_id, 0)
        if consumed:
            scheduler.on_prefill_chunk(request, consumed)
        token = output.tokens.get(request.request_id)
        if token is not None:
            scheduler.on_token(request, token)
    scheduler.end_step()
