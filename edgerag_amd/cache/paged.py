"""Paged KV cache for one sequence, backed by the HIP slot-mapped append and gather kernels.

Interface and pool layout follow the reference ``PagedKVCache`` (``edgerag/cache/paged.py``):
head-major pools ``(kv_heads, num_blocks, block_size, head_dim)`` per layer, shared by every
sequence of an executor; ``update(key, value, layer_idx) -> (keys, values)`` grows the table and
splits shared blocks once per forward, on ``first_layer`` (``:121-149``, ``:151-182``);
``gather`` returns exactly ``seq_len`` tokens so the final block's slack never reaches attention
(``:208-238``).

What changes underneath:

* ``_write`` is one ``edgerag_kv_append`` launch per pool (bit-exact scatter, ``:186-206``); the
  slot mapping is computed on the host from the table and uploaded once per forward and reused by
  every layer, instead of a ``torch.tensor(table.blocks)`` upload per call.
* ``gather`` is one ``edgerag_kv_gather`` launch (the materialised history is still returned,
  because that is this method's contract).
* :meth:`attend` is the fused path: decode attention straight out of the pool via
  ``edgerag_paged_attention``, with no gather copy at all.
* the copy-on-write content copy is ``edgerag_kv_copy_blocks`` over every layer's pool.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from edgerag_amd import kernels
from edgerag_amd.cache.allocator import BlockAllocator
from edgerag_amd.cache.block_table import BlockTable
from edgerag_amd.core.spec import ModelSpec


class PagedKVCache:
    def __init__(
        self,
        spec: ModelSpec,
        allocator: BlockAllocator,
        device: torch.device,
        dtype: torch.dtype = torch.float16,
        pool: list[torch.Tensor] | None = None,
        value_pool: list[torch.Tensor] | None = None,
        first_layer: int = 0,
        n_pool_layers: int | None = None,
    ) -> None:
        self.spec = spec
        self.allocator = allocator
        self.device = torch.device(device)
        self.dtype = dtype
        self.table = BlockTable(allocator=allocator)
        self.first_layer = first_layer
        self.n_pool_layers = n_pool_layers if n_pool_layers is not None else spec.n_layers
        shape = (spec.n_kv_heads, allocator.num_blocks, allocator.block_size, spec.head_dim)
        self.key_pool = pool or [
            torch.zeros(shape, dtype=dtype, device=self.device) for _ in range(self.n_pool_layers)
        ]
        self.value_pool = value_pool or [
            torch.zeros(shape, dtype=dtype, device=self.device) for _ in range(self.n_pool_layers)
        ]
        self._pending_tokens = 0
        # Device metadata of the current forward, shared by every layer.
        self._slots: torch.Tensor | None = None
        self._blocks: torch.Tensor | None = None

    def _pool_index(self, layer_idx: int) -> int:
        return layer_idx - self.first_layer

    # --- interface shared with the reference caches -------------------------------------------

    @property
    def seq_len(self) -> int:
        return self.table.num_tokens

    @property
    def nbytes(self) -> int:
        per_block = self.allocator.block_size * self.spec.n_kv_heads * self.spec.head_dim
        itemsize = torch.finfo(self.dtype).bits // 8
        return 2 * self.table.num_blocks * per_block * itemsize * len(self.key_pool)

    def used_bytes(self) -> int:
        if not self.table.num_blocks:
            return 0
        return self.nbytes * self.seq_len // self.table.capacity

    def begin_append(self, n_new: int) -> None:
        """Once-per-forward bookkeeping: grow the table, split shared blocks, upload slots.

        Called implicitly by :meth:`update`/:meth:`append` on ``first_layer``; the executor may
        call it directly before a forward.
        """
        self._pending_tokens = n_new
        slots = self.reserve(n_new)
        blocks = self.table.ids
        self._slots, self._blocks = kernels.upload_int32([slots, blocks], self.device)

    def blocks_to_reserve(self, n_new: int) -> int:
        """Free blocks :meth:`reserve` would take for ``n_new`` more tokens: the fresh blocks past
        the table's capacity plus a private copy of every shared block in the write range."""
        table, bs = self.table, self.allocator.block_size
        fresh = max(0, self.allocator.blocks_needed(self.seq_len + n_new) - table.num_blocks)
        first, last = self.seq_len // bs, min(table.num_blocks, -(-(self.seq_len + n_new) // bs))
        return fresh + self.allocator.shared_count(table.ids[first:last])

    def reserve(self, n_new: int) -> np.ndarray:
        """Grow the table by ``n_new`` tokens, copy-on-write any shared block in the write range
        (every layer), and return the int32 pool slots of positions ``[seq_len - n_new,
        seq_len)``. The host half of :meth:`begin_append`, for callers that upload several
        sequences' metadata at once (the ragged executor)."""
        self.table.append(n_new)
        try:
            self._unshare_write_range(self.seq_len - n_new, n_new)
        except Exception:
            self.table.shrink_to(self.seq_len - n_new)
            raise
        return self.table.slots(self.seq_len - n_new, n_new)

    def unreserve(self, n_new: int) -> None:
        """Take back the last :meth:`reserve` of ``n_new`` tokens (nothing was written yet)."""
        self.table.shrink_to(self.seq_len - n_new)

    def adopt_prefix(self, blocks: list[int], n_tokens: int) -> None:
        """Start an empty sequence from ``blocks`` (already owned by the caller, e.g. a prefix
        cache hit) holding its first ``n_tokens`` tokens."""
        self.table.adopt(blocks, n_tokens)

    def append(self, key: torch.Tensor, value: torch.Tensor, layer_idx: int) -> None:
        """Write this step's post-RoPE K/V ``(1, kv_heads, n_new, head_dim)``; no gather."""
        if key.shape[0] != 1:
            raise NotImplementedError(
                "PagedKVCache holds one sequence; the ragged executor batches requests"
            )
        n_new = key.shape[2]
        if layer_idx == self.first_layer:
            self.begin_append(n_new)
        if self._slots is None or n_new != self._pending_tokens:
            raise RuntimeError(
                f"layer {layer_idx} appends {n_new} tokens but the forward began with "
                f"{self._pending_tokens}; layer {self.first_layer} must be written first"
            )
        idx = self._pool_index(layer_idx)
        self._write(self.key_pool[idx], key, self.value_pool[idx], value)

    def update(
        self, key: torch.Tensor, value: torch.Tensor, layer_idx: int
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Append, then return the full ``(1, kv_heads, seq_len, head_dim)`` history."""
        self.append(key, value, layer_idx)
        return self.gather(layer_idx)

    def attend(
        self, query: torch.Tensor, layer_idx: int, scaling: float, n_rep: int = 1
    ) -> torch.Tensor:
        """Fused decode attention of ``query (1, n_q_heads, 1, head_dim)`` over this sequence."""
        from edgerag_amd.cache.fused import fused_paged_attention

        idx = self._pool_index(layer_idx)
        block_ids = self._blocks if self._blocks is not None else self._device_blocks()
        return fused_paged_attention(
            query, self.key_pool[idx], self.value_pool[idx], block_ids, self.seq_len, scaling,
            n_rep,
        )

    def _unshare_write_range(self, start: int, n_new: int) -> None:
        """Copy-on-write every shared block in ``[start, start + n_new)``, in every layer's pool."""
        if not self.table.num_blocks or n_new <= 0:
            return
        bs = self.allocator.block_size
        first, last = start // bs, min(self.table.num_blocks, (start + n_new - 1) // bs + 1)
        if not self.allocator.shared_count(self.table.ids[first:last]):
            return  # the usual case: nothing in the write range is shared
        pairs = []
        try:
            for logical in range(first, last):
                copied = self.table.unshare(logical)
                if copied is not None:
                    pairs.append(copied)
        finally:  # a block already switched to its private copy gets its contents either way
            if pairs:
                self._copy_blocks(pairs)

    def _copy_blocks(self, pairs: list[tuple[int, int]]) -> None:
        src, dst = kernels.upload_int32(
            [np.array([p[0] for p in pairs], np.int32), np.array([p[1] for p in pairs], np.int32)],
            self.device,
        )
        for layer in range(len(self.key_pool)):
            kernels.kv_copy_blocks(self.key_pool[layer], src, dst)
            kernels.kv_copy_blocks(self.value_pool[layer], src, dst)

    # --- block-level primitives ---------------------------------------------------------------

    def _write(
        self,
        key_pool: torch.Tensor,
        key: torch.Tensor,
        value_pool: torch.Tensor | None = None,
        value: torch.Tensor | None = None,
    ) -> None:
        """Scatter ``(1, kv_heads, n_new, head_dim)`` sources into their slots (one launch)."""
        k = key[0].transpose(0, 1)  # (n_new, kv_heads, head_dim) view, head_dim contiguous
        v = value[0].transpose(0, 1) if value is not None else None
        if k.stride(2) != 1:
            k = k.contiguous()
        if v is not None and (v.stride() != k.stride()):
            v = v.contiguous()
            k = k.contiguous()
        kernels.kv_append(k, v, self._slots, key_pool, value_pool)

    def _device_blocks(self) -> torch.Tensor:
        (blocks,) = kernels.upload_int32(
            [self.table.ids], self.device
        )
        return blocks

    def gather(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The sequence's K and V as contiguous ``(1, kv_heads, seq_len, head_dim)``."""
        if not self.table.num_blocks or self.seq_len == 0:
            empty = torch.zeros(
                (1, self.spec.n_kv_heads, 0, self.spec.head_dim), dtype=self.dtype,
                device=self.device,
            )
            return empty, empty
        block_ids = self._blocks if self._blocks is not None else self._device_blocks()
        idx = self._pool_index(layer_idx)
        keys = kernels.kv_gather(self.key_pool[idx], block_ids, self.seq_len)
        values = kernels.kv_gather(self.value_pool[idx], block_ids, self.seq_len)
        return keys.unsqueeze(0), values.unsqueeze(0)

    # --- sharing ------------------------------------------------------------------------------

    def fork(self) -> PagedKVCache:
        child = PagedKVCache(
            self.spec, self.allocator, self.device, self.dtype, pool=self.key_pool,
            value_pool=self.value_pool, first_layer=self.first_layer,
        )
        child.table = self.table.fork()
        return child

    def free(self) -> int:
        self._slots = self._blocks = None
        return self.table.free()

    def reset(self) -> None:
        self.free()
        self._pending_tokens = 0

    def blocks_for(self, n_tokens: int) -> int:
        return math.ceil(n_tokens / self.allocator.block_size)
