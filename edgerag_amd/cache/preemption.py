"""Preemption of live sequences when the paged pool runs out: swap, recompute or reject.

Follows ``edgerag/cache/preemption.py`` (``Preemptor`` ``:91-233``): the same policies, records,
statistics, victim order and ``to_dict`` keys. The pools here are head-major
``(kv_heads, num_blocks, block_size, head_dim)`` device tensors, so a victim's KV is the block-axis
slice ``pool[:, blocks]`` of every layer.

* ``swap_out`` gathers the victim's blocks of every layer (one ``index_select`` per pool) and
  copies them into host memory allocated pinned (never registered after the fact), all enqueued
  on the current stream, *then* returns the blocks to the allocator: any later kernel that reuses
  a block is enqueued behind the gather on that stream, so the reference's copy-before-free rule
  (``:119-121``) holds without a host wait. An event marks the copies' end.
* ``swap_in`` reallocates the blocks (``OutOfBlocksError`` when the pool cannot take the sequence
  back: an admission decision, ``:145-149``), waits on the swap-out event, and scatters each layer
  back with one ``index_copy_`` (``:142-171``).

One deliberate difference: the reference reads the block count of a record from axis 0 of the
head-major slice (``:157``, and ``preempt`` returns ``len(record.keys[0])``, ``:186``), which is
the KV-head count; here it is the block axis, so a sequence comes back with as many blocks as it
left with, and ``preempt`` returns the blocks it freed.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from typing import Any

import torch

from edgerag_amd.cache.allocator import BlockAllocator


class PreemptionPolicy(str, Enum):
    """``edgerag/cache/preemption.py:45-48``."""

    SWAP = "swap"
    RECOMPUTE = "recompute"
    REJECT = "reject"


@dataclass
class SwappedSequence:
    """A victim's KV in host memory: per layer ``(kv_heads, n_blocks, block_size, head_dim)``, the
    pool's own layout, so restoring is one scatter per layer."""

    request_id: str
    num_tokens: int
    keys: list[torch.Tensor]
    values: list[torch.Tensor]
    ready: torch.cuda.Event | None = None  # recorded after the device-to-host copies

    @property
    def num_blocks(self) -> int:
        return int(self.keys[0].shape[1])

    @property
    def nbytes(self) -> int:
        per = self.keys[0].numel() * self.keys[0].element_size()
        return 2 * per * len(self.keys)

    def wait(self) -> None:
        """Block the host until the copies have landed (before reading ``keys``/``values``)."""
        if self.ready is not None:
            self.ready.synchronize()


@dataclass
class PreemptionStats:
    preemptions: int = 0
    swaps_out: int = 0
    swaps_in: int = 0
    recomputes: int = 0
    rejects: int = 0
    bytes_swapped: int = 0
    blocks_reclaimed: int = 0
    extra: dict[str, Any] = field(default_factory=dict)


class Preemptor:
    """Frees pool capacity by evicting live sequences under the configured policy."""

    def __init__(self, allocator: BlockAllocator,
                 policy: PreemptionPolicy = PreemptionPolicy.SWAP,
                 pin_memory: bool = True) -> None:
        self.allocator = allocator
        self.policy = PreemptionPolicy(policy)
        # Pinned host memory makes the copies DMA transfers; it is allocated pinned, and the
        # scheduler bounds how many sequences sit swapped (pinned memory is not pageable).
        self.pin_memory = pin_memory and torch.cuda.is_available()
        self.swapped: dict[str, SwappedSequence] = {}
        self.stats = PreemptionStats()

    def _host(self, like: torch.Tensor) -> torch.Tensor:
        return torch.empty(like.shape, dtype=like.dtype, device="cpu",
                           pin_memory=self.pin_memory and like.is_cuda)

    def swap_out(self, request_id: str, blocks: list[int], num_tokens: int,
                 key_pool: list[torch.Tensor], value_pool: list[torch.Tensor]) -> SwappedSequence:
        """Copy a victim's blocks of every layer to host memory, then release the blocks."""
        if request_id in self.swapped:
            raise KeyError(f"{request_id!r} is already swapped out")
        device = key_pool[0].device
        idx = torch.as_tensor(blocks, dtype=torch.long).to(device)
        keys, values = [], []
        for kp, vp in zip(key_pool, value_pool, strict=True):
            for pool, out in ((kp, keys), (vp, values)):
                staged = pool.index_select(1, idx)  # (kv_heads, n_blocks, bs, d), on the stream
                host = self._host(staged)
                host.copy_(staged, non_blocking=host.is_pinned())
                out.append(host)
        ready = None
        if device.type == "cuda":
            ready = torch.cuda.Event()
            ready.record(torch.cuda.current_stream(device))
        record = SwappedSequence(request_id, num_tokens, keys, values, ready)
        self.swapped[request_id] = record
        reclaimed = self.allocator.free(blocks)
        self.stats.preemptions += 1
        self.stats.swaps_out += 1
        self.stats.bytes_swapped += record.nbytes
        self.stats.blocks_reclaimed += reclaimed
        return record

    def swap_in(self, request_id: str, key_pool: list[torch.Tensor],
                value_pool: list[torch.Tensor]) -> tuple[list[int], int]:
        """Reallocate blocks and restore a swapped sequence. Returns ``(blocks, num_tokens)``;
        ``OutOfBlocksError`` (nothing changed) when the pool cannot take it back."""
        record = self.swapped.get(request_id)
        if record is None:
            raise KeyError(f"no swapped sequence {request_id!r}")
        blocks = self.allocator.allocate(record.num_blocks)
        device = key_pool[0].device
        if record.ready is not None and device.type == "cuda":
            torch.cuda.current_stream(device).wait_event(record.ready)
        idx = torch.as_tensor(blocks, dtype=torch.long).to(device)
        for layer, (kp, vp) in enumerate(zip(key_pool, value_pool, strict=True)):
            for pool, host in ((kp, record.keys[layer]), (vp, record.values[layer])):
                pool.index_copy_(1, idx, host.to(device, non_blocking=host.is_pinned()))
        del self.swapped[request_id]
        self.stats.swaps_in += 1
        self.stats.bytes_swapped += record.nbytes
        return blocks, record.num_tokens

    def preempt(self, request_id: str, blocks: list[int], num_tokens: int,
                key_pool: list[torch.Tensor] | None = None,
                value_pool: list[torch.Tensor] | None = None) -> int:
        """Apply the configured policy. Returns the blocks returned to the pool."""
        if self.policy is PreemptionPolicy.SWAP:
            if key_pool is None or value_pool is None:
                raise ValueError("SWAP requires the KV pools")
            before = self.stats.blocks_reclaimed
            self.swap_out(request_id, blocks, num_tokens, key_pool, value_pool)
            return self.stats.blocks_reclaimed - before
        reclaimed = self.allocator.free(blocks)
        self.stats.preemptions += 1
        self.stats.blocks_reclaimed += reclaimed
        if self.policy is PreemptionPolicy.RECOMPUTE:
            self.stats.recomputes += 1
        else:
            self.stats.rejects += 1
        return reclaimed

    @staticmethod
    def select_victims(candidates: list[tuple[str, int]], blocks_needed: int) -> list[str]:
        """Newest first until ``blocks_needed`` is covered (``candidates`` in arrival order), as
        ``edgerag/cache/preemption.py:198-217``."""
        victims: list[str] = []
        freed = 0
        for request_id, held in reversed(candidates):
            if freed >= blocks_needed:
                break
            victims.append(request_id)
            freed += held
        return victims

    @property
    def swapped_bytes(self) -> int:
        return sum(record.nbytes for record in self.swapped.values())

    def to_dict(self) -> dict[str, Any]:
        return {
            "policy": self.policy.value,
            "pin_memory": self.pin_memory,
            "num_swapped": len(self.swapped),
            "swapped_bytes": self.swapped_bytes,
            "preemptions": self.stats.preemptions,
            "swaps_out": self.stats.swaps_out,
            "swaps_in": self.stats.swaps_in,
            "recomputes": self.stats.recomputes,
            "rejects": self.stats.rejects,
            "bytes_swapped": self.stats.bytes_swapped,
            "blocks_reclaimed": self.stats.blocks_reclaimed,
        }
