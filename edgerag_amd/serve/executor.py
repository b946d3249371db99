"""The batch executor: one packed ragged forward per scheduler iteration.

Contract of the reference ``ModelExecutor`` (``edgerag/serve/executor.py:57-156``):
``execute(batch) -> StepOutput``, where each prefilling request advances by at most
``chunk_size`` prompt tokens (``:116-130``), the final prefill chunk emits the request's first
generated token (``:131-136``), each decoding request feeds its last generated token and emits the
next (``:138-154``), a request's ``prompt_embeds`` replace the embedding lookup of its prompt
(``:103-110``), and one KV arena is allocated once and shared by every request's block table
(``:76-83``). Greedy selection is ``argmax`` over the last position's logits.

What changes: the reference runs one decoder forward per request per iteration, each with its own
host-to-device index uploads and a device-to-host argmax. Here the whole batch is one forward:
the host builds the step's metadata (token ids, logical positions, pool slots, cu_seqlens,
context lengths, block tables, the attention work plan, the rows whose logits are read) and
uploads it in one pinned copy; the argmax of every emitting request comes back in one copy.

Requests are duck-typed: this package's :class:`~edgerag_amd.sched.request.Request` (which can
re-feed generated tokens after a recompute preemption) or the reference's own ``Request``
(``edgerag/sched/request.py:37-172``: ``request_id``, ``prompt_token_ids``, ``prompt_embeds``,
``prefill_offset``, ``generated_token_ids``, ``cache``), whose prefill is just its prompt.

A step either happens entirely or not at all on the host side: positions past the model's RoPE
table are refused (``ValueError``) and the batch's block need (fresh blocks plus copy-on-write
copies) is checked against the free pool (:class:`StepDoesNotFit`, an ``OutOfBlocksError``)
before any table changes, so a refused step leaves every request as it was. With a
:class:`~edgerag_amd.cache.prefix.PrefixCache`, a request's first chunk starts after the longest
prefix of full prompt blocks already computed by an earlier request, and a finished prompt's full
blocks are indexed for later ones.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

from edgerag_amd import kernels
from edgerag_amd.cache.allocator import BlockAllocator, OutOfBlocksError
from edgerag_amd.cache.block_table import pack_tables
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


class StepDoesNotFit(OutOfBlocksError):
    """The batch needs more free blocks than the pool has; nothing was changed.
    ``blocks_needed`` is the free count the step needs (pass it to ``Scheduler.preempt``)."""

    def __init__(self, message: str, blocks_needed: int) -> None:
        super().__init__(message)
        self.blocks_needed = blocks_needed


def _prefill_len(request) -> int:
    """Positions a request prefills: its prompt, plus any generated tokens it re-feeds."""
    n = getattr(request, "prefill_len", None)
    return len(request.prompt_token_ids) if n is None else n


def _prefill_ids(request, start: int, end: int) -> list[int]:
    """Token ids of prefill positions ``[start, end)``."""
    take = getattr(request, "prefill_ids", None)
    if take is not None:
        return take(start, end)
    return [int(t) for t in request.prompt_token_ids[start:end]]


def _refeeds(request) -> bool:
    return bool(getattr(request, "refeed", 0))


@dataclass
class _Entry:
    request: Request
    cache: PagedKVCache
    ids: list[int]
    start: int  # first prefill position of the slice (prefill), or the decode position
    consumed: int  # prefill positions this step accounts for (prefix reuse included)
    emits: bool
    prefill: bool


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
        prefix_cache: Any = None,
    ) -> None:
        """``decode_graphs``: replay decode-only iterations (up to ``max_decode_batch`` requests)
        from HIP graphs captured per batch size; iterations with a prefill chunk run eagerly.
        ``prefix_cache``: reuse computed prompt blocks across requests (token-id prompts)."""
        if chunk_size <= 0:
            raise ValueError(f"chunk_size must be positive, got {chunk_size}")
        self.decoder = decoder
        self.spec = spec
        self.allocator = allocator
        self.device = torch.device(device)
        self.dtype = dtype
        self.chunk_size = chunk_size
        self.prefix_cache = prefix_cache
        self.max_positions = spec.max_position_embeddings
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
        # Decode graphs by (requests, attention launch mode of the staged plan).
        self._graphs: dict[tuple[int, int],
                           tuple[torch.cuda.CUDAGraph, torch.Tensor, torch.Tensor]] = {}
        self.graph_steps = 0
        # Tokens come back through a pinned buffer: a direct DMA copy, where a pageable
        # destination goes through a staging copy (batch-1 decode iteration 0.960-0.966 ->
        # 0.934-0.948 ms).
        self._tokens_host = (torch.empty(max(max_decode_batch, 64), dtype=torch.int32,
                                         pin_memory=True)
                             if self.device.type == "cuda" else None)

    @property
    def pool_bytes(self) -> int:
        per_tensor = self.key_pool[0].numel() * self.key_pool[0].element_size()
        return per_tensor * len(self.key_pool) * 2

    def _cache_for(self, request: Request) -> PagedKVCache:
        if request.cache is None:
            request.cache = PagedKVCache(self.spec, self.allocator, self.device, self.dtype,
                                         pool=self.key_pool, value_pool=self.value_pool)
        return request.cache

    # --- host side of a step ------------------------------------------------------------------

    def _entries(self, batch: Batch) -> list[_Entry]:
        entries: list[_Entry] = []
        for request in batch.prefill:
            cache = self._cache_for(request)
            start = request.prefill_offset
            if cache.seq_len != start:
                raise RuntimeError(
                    f"{request.request_id}: cache holds {cache.seq_len} positions but the prompt "
                    f"is read up to {start}"
                )
            total = _prefill_len(request)
            end = min(start + self.chunk_size, total)
            if end > start:
                entries.append(_Entry(request, cache, _prefill_ids(request, start, end), start,
                                      end - start, end >= total, True))
        for request in batch.decode:
            if not request.generated_token_ids:
                raise RuntimeError(
                    f"{request.request_id} is decoding but has no generated token to feed: its "
                    "prefill never emitted one"
                )
            cache = self._cache_for(request)
            entries.append(_Entry(request, cache, [request.generated_token_ids[-1]],
                                  cache.seq_len, 0, True, False))
        return entries

    def _reuse_prefix(self, e: _Entry) -> int:
        """Start a fresh token-id prompt after its longest cached prefix (at least one prompt
        token is left to compute: the first generated token comes out of that forward)."""
        r = e.request
        if (self.prefix_cache is None or not e.prefill or e.start != 0 or _refeeds(r)
                or r.prompt_embeds is not None or e.cache.seq_len):
            return 0
        prompt_len = len(r.prompt_token_ids)
        blocks, n = self.prefix_cache.lookup(r.prompt_token_ids, max_tokens=prompt_len - 1)
        if n:
            e.cache.adopt_prefix(blocks, n)
            total = _prefill_len(r)
            end = min(n + self.chunk_size, total)
            e.ids, e.start = _prefill_ids(r, n, end), n
            e.consumed, e.emits = end, end >= total
        return n

    def _reserve(self, entries: list[_Entry]) -> list[np.ndarray]:
        """All of the step's reservations or none (see the module docstring)."""
        adopted = ([e for e in entries if e.prefill and self._reuse_prefix(e)]
                   if self.prefix_cache is not None else [])

        def undo_adoptions() -> None:
            for e in adopted:
                e.cache.free()
                total = _prefill_len(e.request)
                end = min(self.chunk_size, total)
                e.ids, e.start = _prefill_ids(e.request, 0, end), 0
                e.consumed, e.emits = end, end >= total

        for e in entries:
            top = e.cache.seq_len + len(e.ids)
            if top > self.max_positions:
                undo_adoptions()
                raise ValueError(
                    f"{e.request.request_id}: position {top - 1} is past the model's "
                    f"{self.max_positions} positions (RoPE table)"
                )
        need = sum(e.cache.blocks_to_reserve(len(e.ids)) for e in entries)
        if need > self.allocator.num_free:
            undo_adoptions()
            raise StepDoesNotFit(
                f"step needs {need} free blocks, the pool has {self.allocator.num_free}", need)
        done: list[_Entry] = []
        slots = []
        try:
            for e in entries:
                slots.append(e.cache.reserve(len(e.ids)))
                done.append(e)
        except Exception:
            for e in reversed(done):
                e.cache.unreserve(len(e.ids))
            undo_adoptions()
            raise
        return slots

    def _prompt_rows(self, entries: list[_Entry], qsl: list[int],
                     ids_d: torch.Tensor) -> torch.Tensor | None:
        """Packed input rows when a prefill slice comes with ``prompt_embeds`` (None: every row is
        an embedding lookup)."""
        with_embeds = [(i, e) for i, e in enumerate(entries)
                       if e.prefill and e.request.prompt_embeds is not None]
        if not with_embeds:
            return None
        hidden = self.decoder.embed_tokens[ids_d.long()]
        for i, e in with_embeds:
            pe = e.request.prompt_embeds
            pe = pe[0] if pe.dim() == 3 else pe
            lo, hi = e.start, min(e.start + len(e.ids), len(e.request.prompt_token_ids))
            if hi > lo:
                hidden[qsl[i] : qsl[i] + hi - lo] = pe[lo:hi].to(self.device, self.dtype)
        return hidden

    @torch.inference_mode()
    def execute(self, batch: Batch) -> StepOutput:
        output = StepOutput()
        entries = self._entries(batch)
        if not entries:
            return output
        slots = self._reserve(entries)
        if (self.decode_graphs and not batch.prefill and len(entries) <= self.max_decode_batch
                and self._stage_decode(entries, slots)):
            # One token per request, each emitting: the staging buffer takes the step's lists
            # as they are (no packed arrays are built on the host).
            logits, choice = self._replay_decode(len(entries))
            self.last_logits = logits
            self.graph_steps += 1
            for e, token in zip(entries, self._read_tokens(choice)):
                output.tokens[e.request.request_id] = int(token)
            return output
        qsl, ctx, pos, ids, rows, emitting = [0], [], [], [], [], []
        for e in entries:
            n, L = len(e.ids), e.cache.seq_len
            qsl.append(qsl[-1] + n)
            ctx.append(L)
            pos.append(np.arange(L - n, L, dtype=np.int32))
            ids.extend(e.ids)
            if e.emits:
                rows.append(qsl[-1] - 1)
                emitting.append(e.request)
        bt = pack_tables([e.cache.table for e in entries])
        spec = self.spec
        extras = [np.concatenate(slots).astype(np.int32), np.concatenate(pos),
                  np.asarray(ids, np.int32), np.asarray(rows, np.int32)]
        plan, (slot_d, pos_d, ids_d, rows_d) = kernels.plan_attention(
            np.asarray(qsl, np.int32), np.asarray(ctx, np.int32), bt, spec.n_q_heads,
            spec.n_kv_heads, spec.head_dim, self.allocator.block_size, self.dtype,
            self.device, extras,
        )
        step = StepInputs(ids_d, pos_d, slot_d, rows_d, plan,
                          self._prompt_rows(entries, qsl, ids_d))
        tokens = []
        if emitting:
            logits, choice = self.decoder.greedy(step, self.key_pool, self.value_pool)
            self.last_logits = logits
            tokens = self._read_tokens(choice)
        else:
            self.decoder.forward_hidden(step, self.key_pool, self.value_pool)
        for request, token in zip(emitting, tokens):
            output.tokens[request.request_id] = int(token)
        for e in entries:
            if e.prefill:
                output.prefilled[e.request.request_id] = e.consumed
                if e.emits and self.prefix_cache is not None and not _refeeds(e.request) \
                        and e.request.prompt_embeds is None:
                    self.prefix_cache.register(e.request.prompt_token_ids, e.cache.table.blocks)
        return output

    def _read_tokens(self, choice: torch.Tensor) -> list[int]:
        """The step's greedy tokens on the host (waits for the step)."""
        if self._tokens_host is None or choice.dtype != torch.int32:
            return choice.cpu().tolist()
        n = choice.numel()
        if n > self._tokens_host.numel():
            self._tokens_host = torch.empty(n, dtype=torch.int32, pin_memory=True)
        host = self._tokens_host[:n]
        host.copy_(choice, non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()
        return host.tolist()

    # --- decode iterations replayed from HIP graphs ------------------------------------------

    def _stage_decode(self, entries: list[_Entry], slots: list[np.ndarray]) -> bool:
        """Stage a decode-only step (one token per request) for graph replay; False if it
        does not fit the fixed capacities (the step then runs eagerly)."""
        fx = self._fixed
        if fx is None:
            spec = self.spec
            max_blocks = -(-spec.max_position_embeddings // self.allocator.block_size)
            cap = self.max_decode_batch
            fx = self._fixed = kernels.FixedAttention(
                self.device, spec.n_q_heads, spec.n_kv_heads, spec.head_dim,
                self.allocator.block_size, self.dtype, cap, max_blocks, [cap, cap, cap, cap])
        ctx = [e.cache.seq_len for e in entries]
        n = len(entries)
        extras = [[int(s[0]) for s in slots], [L - 1 for L in ctx], [e.ids[0] for e in entries],
                  fx._arange[:n]]
        return fx.update(None, ctx, [e.cache.table.ids for e in entries], extras)

    def _replay_decode(self, n: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Logits ``(n, vocab)`` of a staged decode-only step of ``n`` requests and their greedy
        tokens (int32 ``(n,)``), both computed inside the replayed graph."""
        fx = self._fixed
        key = (n, *fx.mode)
        entry = self._graphs.get(key)
        if entry is None:
            slots, pos, ids, rows = (e[:n] for e in fx.extras)
            step = StepInputs(ids, pos, slots, rows, fx, all_rows=True)
            stream = torch.cuda.Stream(self.device)
            stream.wait_stream(torch.cuda.current_stream(self.device))
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(stream):
                # The staged metadata is already valid, so run once eagerly first (lets torch and
                # hipBLASLt settle their workspaces outside the capture); it computes this step's
                # logits, which the replay below recomputes identically.
                self.decoder.greedy(step, self.key_pool, self.value_pool)
                with torch.cuda.graph(graph, stream=stream):
                    logits, choice = self.decoder.greedy(step, self.key_pool, self.value_pool)
            torch.cuda.current_stream(self.device).wait_stream(stream)
            entry = self._graphs[key] = (graph, logits, choice)
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
        try:
            output = executor.execute(batch)
        except StepDoesNotFit as short:
            # Nothing ran: free blocks by preemption and decide the iteration again.
            if not scheduler.preempt(short.blocks_needed):
                raise
            continue
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
