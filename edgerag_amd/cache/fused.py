"""Fused paged attention: read K/V straight out of the pool, never materialise a gather.

:func:`fused_paged_attention` keeps the reference signature and contract
(``edgerag/cache/fused.py:242-286``): decode only (one query position), head-count check, an empty
sequence returns zeros, output ``(1, 1, n_q_heads, head_dim)`` in the query's dtype, fp32
accumulation, slots at or past ``seq_len`` masked (``BUGS.md`` P-01 in the reference).

It runs the gfx950 split-KV kernel behind ``edgerag_paged_attention`` -- the same kernel the ragged
executor step uses, with a one-request plan. There is no CPU branch: the executable
specification the reference falls back to lives in this repository's test oracle, not here, so
``force_reference=True`` is refused rather than silently timing the wrong thing.

:func:`ragged_paged_attention` is the batched entry point: a packed token-major query tensor with
``query_start_loc`` / ``context_lens`` / per-request block tables, decodes and chunked-prefill
slices mixed in one launch.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from edgerag_amd import kernels

__all__ = ["fused_paged_attention", "ragged_paged_attention"]


def _check_heads(n_q_heads: int, n_kv_heads: int, n_rep: int) -> None:
    if n_q_heads != n_kv_heads * n_rep:
        raise ValueError(f"{n_q_heads} query heads against {n_kv_heads} kv heads at n_rep={n_rep}")


def fused_paged_attention(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    block_ids: torch.Tensor,
    seq_len: int,
    scaling: float,
    n_rep: int = 1,
    force_reference: bool = False,
) -> torch.Tensor:
    """Decode attention for one sequence. ``query`` is ``(1, n_q_heads, 1, head_dim)``."""
    if force_reference:
        raise ValueError(
            "force_reference: edgerag_amd ships only the HIP kernel; the CPU specification is "
            "test infrastructure (oracle/attention.py)"
        )
    if query.dim() != 4 or query.shape[2] != 1:
        raise ValueError(
            "fused paged attention is the decode path: expected 1 query position, got "
            f"{query.shape[2] if query.dim() == 4 else tuple(query.shape)}"
        )
    n_kv_heads, _, block_size, head_dim = key_pool.shape
    n_q_heads = query.shape[1]
    _check_heads(n_q_heads, n_kv_heads, n_rep)
    if seq_len <= 0:
        return torch.zeros((1, 1, n_q_heads, head_dim), dtype=query.dtype, device=query.device)
    n_blocks = math.ceil(seq_len / block_size)
    if block_ids.numel() < n_blocks:
        raise ValueError(f"{seq_len} tokens need {n_blocks} blocks, block_ids holds {block_ids.numel()}")
    kernels.require_device(query, key_pool, value_pool, block_ids)
    table = block_ids.reshape(-1)[:n_blocks].to(torch.int32).reshape(1, n_blocks)
    plan, _ = kernels.plan_attention(
        np.array([0, 1], np.int32), np.array([seq_len], np.int32),
        np.zeros((1, n_blocks), np.int32), n_q_heads, n_kv_heads, head_dim, block_size,
        query.dtype, query.device,
    )
    plan.block_tables = table.contiguous()
    q = query[0, :, 0, :].unsqueeze(0)  # (1 token, n_q_heads, head_dim)
    out = kernels.paged_attention(q, key_pool, value_pool, plan, scaling)
    return out.reshape(1, 1, n_q_heads, head_dim)


def ragged_paged_attention(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    query_start_loc: np.ndarray,
    context_lens: np.ndarray,
    block_tables: np.ndarray,
    scaling: float,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Attention for a packed ragged batch (host metadata; planned and uploaded in one copy).

    ``query``: ``(num_tokens, n_q_heads, head_dim)``; request ``r`` owns tokens
    ``[query_start_loc[r], query_start_loc[r+1])`` and sees ``context_lens[r]`` cached tokens
    (this step's appends included) through ``block_tables[r]``.
    """
    n_kv_heads, _, block_size, head_dim = key_pool.shape
    plan, _ = kernels.plan_attention(
        query_start_loc, context_lens, block_tables, query.shape[1], n_kv_heads, head_dim,
        block_size, query.dtype, query.device,
    )
    return kernels.paged_attention(query, key_pool, value_pool, plan, scaling, out=out)
