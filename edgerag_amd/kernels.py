"""Tensor-level wrappers over the C ABI in ``include/edgerag_amd.h``.

Each function validates shapes, dtypes and devices on the host, takes torch's current stream and
calls exactly one entry point of ``libedgerag_amd.so``. Nothing here computes on the CPU: tensors
must already live on the HIP device.

Metadata for a ragged step (slot mapping, block tables, cu_seqlens, context lengths and the
attention work plan) is built on the host once per step and moved with a single pinned H2D copy
(:func:`upload_int32`), which replaces the reference's per-layer ``torch.tensor(table.blocks)``
uploads (``BUGS.md`` P-06 in the reference; ``edgerag/cache/paged.py:198-199``, ``:222``).
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import numpy as np
import torch

from edgerag_amd import _lib
from edgerag_amd._lib import call, dtype_code, ptr, require_device, stream_ptr  # noqa: F401

__all__ = [
    "AttentionPlan",
    "FixedAttention",
    "rmsnorm",
    "rope_append",
    "silu_mul",
    "dequantize",
    "kv_append",
    "lm_head_argmax",
    "kv_copy_blocks",
    "kv_gather",
    "paged_attention",
    "paged_attention_noalloc",
    "plan_attention",
    "quant_linear",
    "quantize",
    "upload_int32",
]


def upload_int32(arrays: list[np.ndarray], device: torch.device) -> list[torch.Tensor]:
    """Pack int32 host arrays into one pinned buffer, copy it to ``device`` once, return views.

    Each view starts on a 16-element boundary. The copy is asynchronous on the current stream;
    torch's pinned-memory cache keeps the host buffer alive until the copy has completed.
    """
    offsets, total = [], 0
    for a in arrays:
        offsets.append(total)
        total += (int(a.size) + 15) // 16 * 16
    host = torch.empty(max(total, 16), dtype=torch.int32, pin_memory=True)
    host_np = host.numpy()
    for a, off in zip(arrays, offsets):
        host_np[off : off + a.size] = a.reshape(-1)
    dev = host.to(device, non_blocking=True)
    return [dev[off : off + a.size].view(a.shape) for a, off in zip(arrays, offsets)]


# --- KV cache ---------------------------------------------------------------------------------


def _check_pool(pool: torch.Tensor, name: str) -> None:
    if pool.dim() != 4:
        raise ValueError(f"{name} must be (kv_heads, num_blocks, block_size, head_dim)")
    if not pool.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def kv_append(
    key: torch.Tensor | None,
    value: torch.Tensor | None,
    slot_mapping: torch.Tensor,
    key_pool: torch.Tensor | None,
    value_pool: torch.Tensor | None,
) -> None:
    """Scatter ``key``/``value`` ``(tokens, kv_heads, head_dim)`` into their slots.

    ``slot_mapping`` is device int32 ``(tokens,)``: slot = block * block_size + offset, negative
    to skip a token. Head-major pools ``(kv_heads, num_blocks, block_size, head_dim)``.
    """
    pool = key_pool if key_pool is not None else value_pool
    src = key if key is not None else value
    if pool is None or src is None:
        raise ValueError("kv_append needs at least one of key/value with its pool")
    require_device(key, value, slot_mapping, key_pool, value_pool)
    for p, name in ((key_pool, "key_pool"), (value_pool, "value_pool")):
        if p is not None:
            _check_pool(p, name)
            if p.shape != pool.shape or p.dtype != pool.dtype:
                raise ValueError("key_pool and value_pool must match in shape and dtype")
    if key is not None and value is not None:
        if key.shape != value.shape or key.stride() != value.stride() or key.dtype != value.dtype:
            raise ValueError("key and value must share shape, strides and dtype")
    n_heads, num_blocks, block_size, head_dim = pool.shape
    if src.dim() != 3 or src.shape[1] != n_heads or src.shape[2] != head_dim:
        raise ValueError(
            f"source must be (tokens, {n_heads}, {head_dim}), got {tuple(src.shape)}"
        )
    if src.stride(2) != 1:
        raise ValueError("the head_dim axis of the source must be contiguous")
    if slot_mapping.dtype != torch.int32 or slot_mapping.dim() != 1:
        raise ValueError("slot_mapping must be a 1-D int32 tensor")
    if slot_mapping.shape[0] != src.shape[0]:
        raise ValueError(
            f"slot_mapping has {slot_mapping.shape[0]} entries for {src.shape[0]} tokens"
        )
    if not slot_mapping.is_contiguous():
        slot_mapping = slot_mapping.contiguous()
    call(
        "edgerag_kv_append",
        ptr(key), ptr(value), dtype_code(src.dtype), src.stride(0), src.stride(1),
        slot_mapping.data_ptr(), src.shape[0], ptr(key_pool), ptr(value_pool),
        dtype_code(pool.dtype), n_heads, num_blocks, block_size, head_dim,
        stream_ptr(src.device),
    )


def kv_gather(pool: torch.Tensor, block_ids: torch.Tensor, seq_len: int,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """``(kv_heads, seq_len, head_dim)`` history of one sequence, copied out of the pool (into
    ``out`` when given: contiguous, the pool's dtype)."""
    require_device(pool, block_ids, out)
    _check_pool(pool, "pool")
    n_heads, num_blocks, block_size, head_dim = pool.shape
    if out is None:
        out = torch.empty((n_heads, seq_len, head_dim), dtype=pool.dtype, device=pool.device)
    elif (out.shape != (n_heads, seq_len, head_dim) or out.dtype != pool.dtype
          or not out.is_contiguous()):
        raise ValueError(f"out must be contiguous ({n_heads}, {seq_len}, {head_dim}) {pool.dtype}")
    if seq_len == 0:
        return out
    if block_ids.dtype != torch.int32:
        block_ids = block_ids.to(torch.int32)
    block_ids = block_ids.contiguous()
    need = math.ceil(seq_len / block_size)
    if block_ids.numel() < need:
        raise ValueError(f"{seq_len} tokens need {need} blocks, got {block_ids.numel()}")
    call(
        "edgerag_kv_gather", pool.data_ptr(), dtype_code(pool.dtype), n_heads, num_blocks,
        block_size, head_dim, block_ids.data_ptr(), seq_len, out.data_ptr(),
        stream_ptr(pool.device),
    )
    return out


def kv_copy_blocks(pool: torch.Tensor, src: torch.Tensor, dst: torch.Tensor) -> None:
    """``pool[:, dst[i]] = pool[:, src[i]]`` for every pair (device int32 ids)."""
    require_device(pool, src, dst)
    _check_pool(pool, "pool")
    if src.shape != dst.shape or src.dim() != 1:
        raise ValueError("src and dst must be 1-D and the same length")
    n_heads, num_blocks, block_size, head_dim = pool.shape
    src = src.to(torch.int32).contiguous()
    dst = dst.to(torch.int32).contiguous()
    call(
        "edgerag_kv_copy_blocks", pool.data_ptr(), dtype_code(pool.dtype), n_heads, num_blocks,
        block_size, head_dim, src.data_ptr(), dst.data_ptr(), src.numel(),
        stream_ptr(pool.device),
    )


# --- ragged paged attention -------------------------------------------------------------------


@dataclass
class AttentionPlan:
    """Host plan plus its device copy, and everything the run needs for one step.

    Built once per step and reused by every layer: the metadata is identical across layers.
    """

    plan_host: np.ndarray
    plan_dev: torch.Tensor
    query_start_loc: torch.Tensor
    context_lens: torch.Tensor
    block_tables: torch.Tensor
    workspace: torch.Tensor | None
    workspace_bytes: int
    num_reqs: int
    num_tokens: int
    n_q_heads: int
    n_kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype

    @property
    def n_items(self) -> int:
        return int(self.plan_host[2])

    @property
    def decode_only(self) -> bool:
        """Every work item is a decode row (no prefill tiles): the append can fuse in."""
        return int(self.plan_host[2]) == int(self.plan_host[13])

    @property
    def overlap_rows(self) -> bool:
        """The planner sized this batch's prefill tiles to run beside its decode rows on a second
        stream (both are heavy, or ``force_overlap`` asked for it); else one stream runs all."""
        return int(self.plan_host[_lib.PLAN_WORD_OVERLAP]) == 1


_WORKSPACES: dict[torch.device, torch.Tensor] = {}


def attention_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A per-device attention workspace (split partials) of at least ``nbytes``, reused across
    steps so a step allocates nothing. Launches that share it must be ordered on one stream,
    which is how the executor and the benchmark use it."""
    device = torch.device(device)
    buf = _WORKSPACES.get(device)
    if buf is None or buf.numel() < nbytes:
        size = max(nbytes, 2 * buf.numel() if buf is not None else 0, 1 << 20)
        buf = torch.empty(size, dtype=torch.uint8, device=device)
        _WORKSPACES[device] = buf
    return buf


_QUANT_WORKSPACES: dict[torch.device, torch.Tensor] = {}


def quant_workspace(device: torch.device) -> torch.Tensor:
    """The per-device split-K workspace of the quant linears: the largest any shape uses,
    allocated once and never replaced (a HIP graph that captured a launch keeps using the same
    buffer). Launches that share it must be ordered on one stream."""
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    buf = _QUANT_WORKSPACES.get(device)
    if buf is None:
        buf = torch.empty(_lib.QUANT_WORKSPACE_MAX, dtype=torch.uint8, device=device)
        _QUANT_WORKSPACES[device] = buf
    return buf


def quant_workspace_bytes(m: int, k: int, n: int, bits: int, group_size: int) -> int:
    """Workspace bytes the split-K quant linear uses for this shape (0: it does not split)."""
    return int(_lib.load().edgerag_quant_linear_workspace_bytes(m, k, n, bits, group_size))


_PLAN_WORDS_HINT = [1 << 14]  # largest plan seen so far: one planner call is usually enough


def make_plan_host(
    query_start_loc: np.ndarray,
    context_lens: np.ndarray,
    n_q_heads: int,
    n_kv_heads: int,
    head_dim: int,
    block_size: int,
    max_blocks_per_seq: int,
    dtype: torch.dtype,
    split_rows: bool = False,
    force_overlap: bool = False,
) -> tuple[np.ndarray, int]:
    """Run the native host planner. Returns ``(plan words, workspace bytes)``.

    One planner call fills a buffer sized from the largest plan seen so far; only a plan larger
    than every earlier one needs a second call (the first reports the size). ``split_rows``
    plans decode rows as KV splits merged by a launch (``EDGERAG_PLAN_SPLIT_ROWS``) instead of
    workgroups whose waves merge in LDS. ``force_overlap`` plans any batch with both prefill
    tiles and decode rows for the two-stream run (``EDGERAG_PLAN_OVERLAP``), which the planner
    otherwise picks only when both are heavy."""
    lib = _lib.load()
    qsl = np.ascontiguousarray(query_start_loc, dtype=np.int32)
    ctx = np.ascontiguousarray(context_lens, dtype=np.int32)
    num_reqs = ctx.size
    if qsl.size != num_reqs + 1:
        raise ValueError(f"query_start_loc needs {num_reqs + 1} entries, got {qsl.size}")
    words, ws = ctypes.c_int64(0), ctypes.c_int64(0)
    args = (
        qsl.ctypes.data, ctx.ctypes.data, num_reqs, n_q_heads, n_kv_heads, head_dim, block_size,
        max_blocks_per_seq, dtype_code(dtype),
        (_lib.PLAN_SPLIT_ROWS if split_rows else 0) | (_lib.PLAN_OVERLAP if force_overlap else 0),
    )
    plan = np.empty(_PLAN_WORDS_HINT[0], dtype=np.int32)
    rc = lib.edgerag_attn_plan_ex(*args, plan.ctypes.data, plan.size, ctypes.byref(words),
                                  ctypes.byref(ws))
    if rc == _lib.EDGERAG_EWORKSPACE and words.value > plan.size:
        plan = np.empty(words.value, dtype=np.int32)
        rc = lib.edgerag_attn_plan_ex(*args, plan.ctypes.data, plan.size, ctypes.byref(words),
                                      ctypes.byref(ws))
    if rc != _lib.EDGERAG_OK:
        raise _lib.EdgeragError("edgerag_attn_plan", rc,
                                lib.edgerag_last_error().decode(errors="replace"))
    _PLAN_WORDS_HINT[0] = max(_PLAN_WORDS_HINT[0], int(words.value))
    return plan[: words.value], int(ws.value)


def plan_attention(
    query_start_loc: np.ndarray,
    context_lens: np.ndarray,
    block_tables: np.ndarray,
    n_q_heads: int,
    n_kv_heads: int,
    head_dim: int,
    block_size: int,
    dtype: torch.dtype,
    device: torch.device,
    extra_int32: list[np.ndarray] | None = None,
    workspace: bool = True,
    split_rows: bool = False,
    force_overlap: bool = False,
) -> tuple[AttentionPlan, list[torch.Tensor]]:
    """Plan a ragged step on the host and upload all of its metadata in one copy.

    ``extra_int32`` arrays (e.g. the step's slot mapping) ride along in the same copy; their
    device views are returned second. ``workspace=False`` leaves the split-partial workspace out
    (for :func:`paged_attention_noalloc`, which keeps them in the library's static scratch).
    """
    block_tables = np.ascontiguousarray(block_tables, dtype=np.int32)
    if block_tables.ndim != 2:
        raise ValueError("block_tables must be (num_reqs, max_blocks)")
    plan, ws_bytes = make_plan_host(
        query_start_loc, context_lens, n_q_heads, n_kv_heads, head_dim, block_size,
        block_tables.shape[1], dtype, split_rows, force_overlap,
    )
    extra = list(extra_int32 or [])
    views = upload_int32(
        [plan, np.asarray(query_start_loc, np.int32), np.asarray(context_lens, np.int32),
         block_tables, *extra],
        device,
    )
    ws = attention_workspace(device, ws_bytes) if ws_bytes > 0 and workspace else None
    num_reqs = int(np.asarray(context_lens).size)
    ap = AttentionPlan(
        plan_host=plan, plan_dev=views[0], query_start_loc=views[1], context_lens=views[2],
        block_tables=views[3], workspace=ws, workspace_bytes=ws_bytes, num_reqs=num_reqs,
        num_tokens=int(np.asarray(query_start_loc)[-1]) if num_reqs else 0,
        n_q_heads=n_q_heads, n_kv_heads=n_kv_heads, head_dim=head_dim, block_size=block_size,
        dtype=dtype,
    )
    return ap, views[4:]


def _attention_operands(query, key_pool, value_pool, plan, out):
    """Validate one planned attention launch; returns ``(query, out, leading C-ABI arguments)``:
    everything ``edgerag_paged_attention`` takes before its workspace."""
    require_device(query, key_pool, value_pool)
    _check_pool(key_pool, "key_pool")
    _check_pool(value_pool, "value_pool")
    if key_pool.shape != value_pool.shape or key_pool.dtype != value_pool.dtype:
        raise ValueError("key_pool and value_pool must match")
    n_kv, num_blocks, block_size, head_dim = key_pool.shape
    if query.dim() != 3 or query.shape[1] != plan.n_q_heads or query.shape[2] != head_dim:
        raise ValueError(
            f"query must be (tokens, {plan.n_q_heads}, {head_dim}), got {tuple(query.shape)}"
        )
    if query.dtype != key_pool.dtype:
        raise ValueError(f"query dtype {query.dtype} != pool dtype {key_pool.dtype}")
    if (n_kv, block_size, head_dim, query.dtype) != (
        plan.n_kv_heads, plan.block_size, plan.head_dim, plan.dtype
    ):
        raise ValueError("the attention plan was built for a different pool shape")
    if query.stride(2) != 1:
        query = query.contiguous()
    if out is None:
        out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    elif out.shape != query.shape or out.dtype != query.dtype or out.stride(2) != 1:
        raise ValueError("out must match query in shape and dtype, head_dim contiguous")
    return query, out, (
        plan.plan_host.ctypes.data, plan.plan_dev.data_ptr(), plan.plan_host.size,
        query.data_ptr(), query.stride(0), query.stride(1),
        key_pool.data_ptr(), value_pool.data_ptr(), dtype_code(key_pool.dtype),
        plan.block_tables.data_ptr(), plan.block_tables.stride(0),
        plan.query_start_loc.data_ptr(), plan.context_lens.data_ptr(),
        plan.num_reqs, query.shape[0], plan.n_q_heads, n_kv, head_dim, block_size, num_blocks,
    )


def paged_attention(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    plan: AttentionPlan,
    scale: float,
    out: torch.Tensor | None = None,
    overlap: bool = True,
) -> torch.Tensor:
    """Ragged paged attention. ``query``/``out``: ``(num_tokens, n_q_heads, head_dim)``.

    With ``overlap`` and a plan made for it (:attr:`AttentionPlan.overlap_rows`: heavy prefill
    tiles beside heavy decode rows), the two run on two streams (joined before the split merge),
    so MFMA work overlaps the KV streaming."""
    query, out, lead = _attention_operands(query, key_pool, value_pool, plan, out)
    if plan.workspace_bytes > 0 and plan.workspace is None:
        raise ValueError("this plan was built without a workspace: use paged_attention_noalloc")
    ws = plan.workspace
    args = (*lead, float(scale), out.data_ptr(), out.stride(0), out.stride(1),
            None if ws is None else ws.data_ptr(), plan.workspace_bytes)
    device = query.device
    if overlap and plan.overlap_rows:
        # Prefill tiles (MFMA-bound) beside the decode rows (HBM-bound) on a side stream; the
        # merge of split partials waits for both. The tiles go first, on the current stream (the
        # side stream starts a few microseconds later, after its event wait), at one workgroup per
        # CU: launched second, or at two per CU, they found every CU's registers taken by row
        # waves and ran mostly after the rows.
        main = torch.cuda.current_stream(device)
        side = _side_stream(device)
        fork, join = _overlap_events(device)
        fork.record(main)
        side.wait_event(fork)
        call("edgerag_paged_attention", *args, _lib.ATTN_TILES | _lib.ATTN_TILES_SHARED,
             main.cuda_stream)
        call("edgerag_paged_attention", *args, _lib.ATTN_ROWS, side.cuda_stream)
        join.record(side)
        main.wait_event(join)
        call("edgerag_paged_attention", *args, _lib.ATTN_COMBINE, main.cuda_stream)
    else:
        call("edgerag_paged_attention", *args, _lib.ATTN_ALL, stream_ptr(device))
    return out


def paged_attention_noalloc(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    plan: AttentionPlan,
    scale: float,
    out: torch.Tensor,
    parts: int = _lib.ATTN_ALL,
) -> torch.Tensor:
    """:func:`paged_attention` through ``edgerag_paged_attention_noalloc``: the split partials
    live in the library's static per-GPU scratch (``_lib.ATTN_SCRATCH_BYTES``), so the call
    allocates nothing, ``out`` included (the caller passes it). Calls that overlap in time on one
    GPU share that scratch and must be ordered by the caller (one stream does it)."""
    if out is None:
        raise ValueError("paged_attention_noalloc writes into a caller-provided out")
    query, out, lead = _attention_operands(query, key_pool, value_pool, plan, out)
    call("edgerag_paged_attention_noalloc", *lead, float(scale), out.data_ptr(), out.stride(0),
         out.stride(1), int(parts), stream_ptr(query.device))
    return out


def paged_attention_append(
    key: torch.Tensor,
    value: torch.Tensor,
    slot_mapping: torch.Tensor,
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    plan: AttentionPlan,
    scale: float,
    out: torch.Tensor | None = None,
    overlap: bool = True,
) -> torch.Tensor:
    """``kv_append(key, value, slot_mapping, pools)`` then ``paged_attention(query, ...)``, with the
    same results; one launch for decode batches (the waves reaching a request's new positions read
    them from ``key``/``value`` and write them to the pools). With ``overlap`` and a plan made for
    the two-stream run, the attention after the append overlaps tiles and rows as
    ``paged_attention`` does."""
    require_device(key, value, slot_mapping, query, key_pool, value_pool)
    _check_pool(key_pool, "key_pool")
    _check_pool(value_pool, "value_pool")
    if key_pool.shape != value_pool.shape or key_pool.dtype != value_pool.dtype:
        raise ValueError("key_pool and value_pool must match")
    n_kv, num_blocks, block_size, head_dim = key_pool.shape
    if key.shape != value.shape or key.stride() != value.stride() or key.dtype != value.dtype:
        raise ValueError("key and value must share shape, strides and dtype")
    if key.dim() != 3 or key.shape[1:] != (n_kv, head_dim) or key.stride(2) != 1:
        raise ValueError(f"new K/V must be (tokens, {n_kv}, {head_dim}), head_dim contiguous")
    if slot_mapping.dtype != torch.int32 or slot_mapping.shape != (key.shape[0],):
        raise ValueError("slot_mapping must be int32 with one entry per new token")
    if query.dim() != 3 or query.shape[1] != plan.n_q_heads or query.shape[2] != head_dim:
        raise ValueError(
            f"query must be (tokens, {plan.n_q_heads}, {head_dim}), got {tuple(query.shape)}"
        )
    if key.shape[0] != query.shape[0]:
        raise ValueError("one new K/V row per query token")
    if query.dtype != key_pool.dtype:
        raise ValueError(f"query dtype {query.dtype} != pool dtype {key_pool.dtype}")
    if (n_kv, block_size, head_dim, query.dtype) != (
        plan.n_kv_heads, plan.block_size, plan.head_dim, plan.dtype
    ):
        raise ValueError("the attention plan was built for a different pool shape")
    if query.stride(2) != 1:
        query = query.contiguous()
    if out is None:
        out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    elif out.shape != query.shape or out.dtype != query.dtype or out.stride(2) != 1:
        raise ValueError("out must match query in shape and dtype, head_dim contiguous")
    if overlap and plan.overlap_rows:
        # A batch with prefill tiles: the append, then the tiles and the decode rows overlapped
        # on two streams (paged_attention). Appending only the tiles' rows first and letting the
        # rows append their own positions beside them measured slower (config 3: 0.242-0.26
        # against 0.221 ms per step): the rows then take the CUs before the tiles are resident.
        kv_append(key, value, slot_mapping, key_pool, value_pool)
        return paged_attention(query, key_pool, value_pool, plan, scale, out=out, overlap=True)
    ws = plan.workspace
    call(
        "edgerag_paged_attention_append", key.data_ptr(), value.data_ptr(),
        dtype_code(key.dtype), key.stride(0), key.stride(1), slot_mapping.contiguous().data_ptr(),
        plan.plan_host.ctypes.data, plan.plan_dev.data_ptr(), plan.plan_host.size,
        query.data_ptr(), query.stride(0), query.stride(1),
        key_pool.data_ptr(), value_pool.data_ptr(), dtype_code(key_pool.dtype),
        plan.block_tables.data_ptr(), plan.block_tables.stride(0),
        plan.query_start_loc.data_ptr(), plan.context_lens.data_ptr(),
        plan.num_reqs, query.shape[0], plan.n_q_heads, n_kv, head_dim, block_size, num_blocks,
        float(scale), out.data_ptr(), out.stride(0), out.stride(1),
        None if ws is None else ws.data_ptr(), plan.workspace_bytes, stream_ptr(query.device),
    )
    return out


_OVERLAP_EVENTS: dict = {}
_SIDE_STREAMS: dict[torch.device, torch.cuda.Stream] = {}


def _overlap_events(device: torch.device) -> tuple[torch.cuda.Event, torch.cuda.Event]:
    """Two events per device, made once, that order the side stream after the current one (fork)
    and the current one after the side stream (join). A wait binds to the event's latest record
    when it is enqueued, so recording the same event again for the next call is safe, and no
    event is created per call (torch's wait_stream makes one each time)."""
    device = torch.device(device)
    events = _OVERLAP_EVENTS.get(device)
    if events is None:
        events = _OVERLAP_EVENTS[device] = (torch.cuda.Event(), torch.cuda.Event())
    return events


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """One extra stream per device (default priority) for work that overlaps the current one."""
    device = torch.device(device)
    stream = _SIDE_STREAMS.get(device)
    if stream is None:
        stream = _SIDE_STREAMS[device] = torch.cuda.Stream(device)
    return stream


class FixedAttention:
    """Decode-only ragged attention with a launch shape fixed at construction, for HIP graphs.

    All step metadata lives in one static device buffer, rewritten in place before every replay
    by :meth:`update` (one pinned H2D copy): cu_seqlens, context lengths, block tables with a
    fixed row stride, caller-defined extra int32 arrays (token ids, positions, slots, ...) and the
    plan. :meth:`launch` calls ``edgerag_paged_attention_fixed``, whose grid depends only on the
    capacities and on :attr:`mode`, the launch mode of the staged plan: row waves 0 for KV splits
    merged by a combine launch, > 0 for workgroup-split rows (the planner takes these when every
    context is short and the rows are few, or cuts the contexts into parts when the batch has few
    requests); whether
    a merge launch follows; and the plan's partial slots (parts in fixed slots take the merge
    launch that reads no plan entry first). A captured graph stays valid for every plan
    :meth:`update` accepts in the mode it was captured in, so callers key their graphs by
    :attr:`mode` as well.
    The pinned host staging buffer is reused: the caller must have synchronised with the previous
    step (the executor does, when it reads the tokens back) before calling :meth:`update` again.
    """

    def __init__(self, device, n_q_heads: int, n_kv_heads: int, head_dim: int, block_size: int,
                 dtype: torch.dtype, max_reqs: int, max_blocks_per_seq: int,
                 extra_capacities: list[int], max_items: int = 16384,
                 min_split: int = 256, split_rows: bool = False) -> None:
        """``split_rows``: always plan decode rows as KV splits merged by a launch, never as
        workgroup-split rows."""
        self.device = torch.device(device)
        self.split_rows = split_rows
        self.n_q_heads, self.n_kv_heads, self.head_dim = n_q_heads, n_kv_heads, head_dim
        self.block_size, self.dtype = block_size, dtype
        self.max_reqs, self.max_blocks = max_reqs, max_blocks_per_seq
        self.max_row_vecs = min(8, max(1, n_q_heads // n_kv_heads))
        # Capacities of both launch modes: KV splits (items, merge rows, partials) and
        # workgroup-split rows (one workgroup per request and kv head, or per part of a context
        # when the batch has few requests), the latter bounded by the planner itself.
        self.max_combine = max_reqs
        # Every slot of a slotted plan (at most 32 per token and head) or every split.
        max_splits = max(-(-max_blocks_per_seq * block_size // min(min_split, 128)), 32)
        self.max_partials = max_reqs * n_q_heads * max_splits
        self.max_items = max_items
        self.wg_items = int(_lib.load().edgerag_attn_fixed_row_items(
            max_reqs, n_kv_heads, max_blocks_per_seq * block_size, block_size))
        self.row_waves = 0
        self.combine = False
        self.slots = 0
        self.plan_words = 24 + 8 * max_items + 4 * max_reqs + 8 * self.max_combine + 64

        def pad(n: int) -> int:
            return (n + 15) // 16 * 16

        # Layout: cu_seqlens, context lengths, extras, the block tables, then the plan last, so
        # that a step uploads [0, end of its plan) in one copy.
        sizes = [pad(max_reqs + 1), pad(max_reqs), *[pad(c) for c in extra_capacities],
                 pad(max_reqs * max_blocks_per_seq)]
        offs, at = [], 0
        for n in sizes:
            offs.append(at)
            at += pad(n)
        self._tables_off = offs[-1]
        self._plan_off = at
        total = self._plan_off + self.plan_words
        self.buf = torch.zeros(total, dtype=torch.int32, device=self.device)
        self.host = torch.zeros(total, dtype=torch.int32, pin_memory=True)
        self._host_np = self.host.numpy()
        self._host_np[self._tables_off : self._plan_off] = -1
        self.qsl = self.buf[offs[0] : offs[0] + max_reqs + 1]
        self.ctx = self.buf[offs[1] : offs[1] + max_reqs]
        tables = self._tables_off
        self.block_tables = self.buf[tables : tables + max_reqs * max_blocks_per_seq].view(
            max_reqs, max_blocks_per_seq)
        self.extras = [self.buf[o : o + c] for o, c in zip(offs[2:-1], extra_capacities)]
        self._offs, self._caps = offs[:-1], extra_capacities
        self.plan = self.buf[self._plan_off :]
        acc_off = (self.max_partials * 8 + 255) // 256 * 256
        ws = acc_off + (self.max_partials * head_dim * 4 + 255) // 256 * 256
        self.workspace = torch.empty(ws, dtype=torch.uint8, device=self.device)
        self.num_reqs = 0
        self._table_rows = [0] * max_reqs  # entries written per table row (the rest hold -1)
        # The planner reads cu_seqlens / context lengths from the staging buffer and writes the
        # plan into it: no host array is built or copied per step.
        base = self.host.data_ptr()
        self._plan_fn = _lib.load().edgerag_attn_plan_ex
        self._plan_args = (base + 4 * offs[0], base + 4 * offs[1])
        self._plan_flags = _lib.PLAN_SPLIT_ROWS if split_rows else 0
        self._plan_dst = base + 4 * self._plan_off
        self._words, self._ws = ctypes.c_int64(0), ctypes.c_int64(0)
        self._words_p, self._ws_p = ctypes.byref(self._words), ctypes.byref(self._ws)
        self._arange = np.arange(max_reqs + 1, dtype=np.int32)

    def update(self, query_start_loc: np.ndarray | None, context_lens,
               block_tables, extras: list) -> bool:
        """Plan the step and stage it; False (nothing uploaded) if it exceeds a capacity or has
        prefill tiles -- the caller then runs the eager path. ``query_start_loc`` None: one
        query token per request. ``block_tables``: a ``[R, width]`` int32 array, or one int32
        row per request (each as long as that request's table)."""
        R = len(context_lens)
        if R > self.max_reqs:
            return False
        for e, c in zip(extras, self._caps):
            if len(e) > c:
                return False
        h = self._host_np
        o = self._offs
        h[o[0] : o[0] + R + 1] = self._arange[: R + 1] if query_start_loc is None \
            else query_start_loc
        h[o[1] : o[1] + R] = context_lens
        # Table rows: this step's entries, -1 past them where an earlier step wrote more.
        t0, mb, rows = self._tables_off, self.max_blocks, self._table_rows
        for r in range(R):
            row = block_tables[r]
            n = len(row)
            if n > mb:
                return False
            at = t0 + r * mb
            h[at : at + n] = row
            if rows[r] > n:
                h[at + n : at + rows[r]] = -1
            rows[r] = n
        for e, off in zip(extras, o[2:]):
            h[off : off + len(e)] = e
        rc = self._plan_fn(*self._plan_args, R, self.n_q_heads, self.n_kv_heads, self.head_dim,
                           self.block_size, self.max_blocks, dtype_code(self.dtype),
                           self._plan_flags, self._plan_dst, self.plan_words, self._words_p,
                           self._ws_p)
        if rc == _lib.EDGERAG_EWORKSPACE:
            return False  # the plan does not fit the staging capacity
        if rc != _lib.EDGERAG_OK:
            raise _lib.EdgeragError("edgerag_attn_plan", rc,
                                    _lib.load().edgerag_last_error().decode(errors="replace"))
        po = self._plan_off
        hdr = h[po : po + 22].tolist()
        n_items, n_row, n_partials = hdr[2], hdr[13], hdr[6]
        row_waves, n_combine, slots = hdr[19], hdr[16], hdr[21]
        if (n_items != n_row or n_row > (self.wg_items if row_waves else self.max_items)
                or n_combine > self.max_combine or hdr[14] > self.max_row_vecs
                or n_partials > self.max_partials):
            return False
        used = po + int(self._words.value)
        self.buf[:used].copy_(self.host[:used], non_blocking=True)
        self.num_reqs = R
        self.row_waves = row_waves
        self.combine = n_combine > 0
        self.slots = slots if self.combine else 0
        return True

    @property
    def mode(self) -> tuple[int, bool, int]:
        """The launch shape the staged plan needs: (row waves, merge launch, partial slots). A
        graph captured in one mode replays every plan staged in that mode."""
        return self.row_waves, self.combine, self.slots

    def launch(self, query: torch.Tensor, key_pool: torch.Tensor, value_pool: torch.Tensor,
               scale: float, out: torch.Tensor) -> torch.Tensor:
        n_kv, num_blocks, block_size, head_dim = key_pool.shape
        if query.stride(2) != 1 or out.stride(2) != 1:
            raise ValueError("query and out need a contiguous head_dim axis")
        items = self.wg_items if self.row_waves else self.max_items
        combine, partials = (self.max_combine, self.max_partials) if self.combine else (0, 0)
        call(
            "edgerag_paged_attention_fixed", self.plan.data_ptr(), items, combine,
            self.max_row_vecs, partials, self.row_waves, self.slots, query.data_ptr(),
            query.stride(0), query.stride(1), key_pool.data_ptr(), value_pool.data_ptr(),
            dtype_code(key_pool.dtype), self.block_tables.data_ptr(), self.max_blocks,
            self.qsl.data_ptr(), self.ctx.data_ptr(), self.n_q_heads, n_kv, head_dim, block_size,
            num_blocks, float(scale), out.data_ptr(), out.stride(0), out.stride(1),
            self.workspace.data_ptr(), self.workspace.numel(), stream_ptr(query.device),
        )
        return out


# --- fused layer ops ----------------------------------------------------------------------------


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, delta: torch.Tensor | None = None,
            h_out: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``out = RMSNorm(x (+ delta))`` row-wise over ``(rows, width)``; with ``delta`` the sum
    is also written to ``h_out`` (which may be ``x``)."""
    require_device(x, weight, delta, h_out, out)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("rmsnorm takes (rows, width) with contiguous rows")
    rows, width = x.shape
    if out is None:
        out = torch.empty_like(x)
    if delta is not None:
        if delta.shape != x.shape or delta.stride(1) != 1 or h_out is None:
            raise ValueError("delta must match x, and h_out is required with delta")
    call(
        "edgerag_rmsnorm", x.data_ptr(), x.stride(0), ptr(delta),
        delta.stride(0) if delta is not None else 0, weight.data_ptr(), ptr(h_out),
        h_out.stride(0) if h_out is not None else 0, out.data_ptr(), out.stride(0), rows, width,
        float(eps), dtype_code(x.dtype), stream_ptr(x.device),
    )
    return out


def embed_rmsnorm_fits(table: torch.Tensor) -> bool:
    """Whether :func:`embed_rmsnorm` takes rows of this table: whole 16-byte chunks, at most
    8 x 256 of them, rows 16-byte aligned."""
    width = table.shape[1]
    es = table.element_size()
    return (table.dim() == 2 and table.stride(1) == 1 and (width * es) % 16 == 0
            and width * es // 16 <= 8 * 256 and (table.stride(0) * es) % 16 == 0
            and table.data_ptr() % 16 == 0)


def embed_rmsnorm(ids: torch.Tensor, table: torch.Tensor, weight: torch.Tensor, eps: float,
                  h_out: torch.Tensor | None = None, out: torch.Tensor | None = None,
                  rope: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
                  ) -> tuple[torch.Tensor, torch.Tensor, tuple[torch.Tensor, torch.Tensor] | None]:
    """The embedding rows of the int32 ``ids`` (``h``, a copy of ``table[ids]``) and their
    RMSNorm (``out``), in one launch; returns ``(h, out, rows)``. An id outside the table gives a
    row of NaN in both. ``rope = (positions, cos, sin)``: the same launch also gathers what
    :func:`rope_rows` returns (``rows``; None without ``rope``)."""
    require_device(ids, table, weight, h_out, out)
    if ids.dtype != torch.int32 or ids.dim() != 1 or (ids.numel() > 1 and ids.stride(0) != 1):
        raise ValueError("ids must be a contiguous int32 vector")
    if not embed_rmsnorm_fits(table):
        raise ValueError("embed_rmsnorm takes tables with 16-byte aligned rows of whole 16-byte "
                         "chunks (at most 2,048 of them)")
    rows, (vocab, width) = ids.numel(), table.shape
    if h_out is None:
        h_out = torch.empty((rows, width), device=table.device, dtype=table.dtype)
    if out is None:
        out = torch.empty_like(h_out)
    rope_args, rows_out = (None, None, None, 0, 0, None, None), None
    if rope is not None:
        positions, cos, sin = rope
        require_device(positions, cos, sin)
        if positions.dtype != torch.int32 or positions.numel() != rows or \
                not positions.is_contiguous():
            raise ValueError("positions must be a contiguous int32 vector, one per id")
        if cos.shape != sin.shape or cos.dim() != 2 or not (cos.is_contiguous() and
                                                           sin.is_contiguous()) \
                or cos.dtype != table.dtype or sin.dtype != table.dtype:
            raise ValueError("cos and sin must be matching contiguous (max_pos, head_dim) tables "
                             "of the embedding's dtype")
        c = torch.empty((rows, cos.shape[1]), dtype=cos.dtype, device=cos.device)
        sn = torch.empty_like(c)
        rope_args = (positions.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
                     cos.shape[1], c.data_ptr(), sn.data_ptr())
        rows_out = (c, sn)
    call(
        "edgerag_embed_rmsnorm", ids.data_ptr(), rows, table.data_ptr(), table.stride(0), vocab,
        weight.data_ptr(), h_out.data_ptr(), h_out.stride(0), out.data_ptr(), out.stride(0),
        width, float(eps), *rope_args, dtype_code(table.dtype), stream_ptr(table.device),
    )
    return h_out, out, rows_out


def rope_append(qkv: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                n_q_heads: int, n_kv_heads: int, head_dim: int, slots: torch.Tensor,
                key_pool: torch.Tensor, value_pool: torch.Tensor,
                q_out: torch.Tensor | None = None) -> torch.Tensor:
    """RoPE on the fused projection rows; q returned ``(T, n_q_heads, head_dim)``, post-RoPE k
    and v written into the pools at ``slots``."""
    require_device(qkv, positions, cos, sin, slots, key_pool, value_pool, q_out)
    T = qkv.shape[0]
    if qkv.dim() != 2 or qkv.stride(1) != 1 or qkv.shape[1] != (n_q_heads + 2 * n_kv_heads) * head_dim:
        raise ValueError("qkv must be (tokens, (n_q + 2 n_kv) * head_dim) with contiguous rows")
    for p in (key_pool, value_pool):
        _check_pool(p, "pool")
    nkv, num_blocks, block_size, d = key_pool.shape
    if nkv != n_kv_heads or d != head_dim or cos.shape != sin.shape or cos.shape[1] != head_dim:
        raise ValueError("pool / rotary table shapes do not match the heads")
    if positions.dtype != torch.int32 or slots.dtype != torch.int32:
        raise ValueError("positions and slots must be int32")
    if q_out is None:
        q_out = torch.empty((T, n_q_heads, head_dim), dtype=qkv.dtype, device=qkv.device)
    call(
        "edgerag_rope_append", qkv.data_ptr(), qkv.stride(0), positions.data_ptr(),
        cos.data_ptr(), sin.data_ptr(), cos.shape[0], T, n_q_heads, n_kv_heads, head_dim,
        q_out.data_ptr(), q_out.stride(0), slots.data_ptr(), key_pool.data_ptr(),
        value_pool.data_ptr(), num_blocks, block_size, dtype_code(qkv.dtype),
        stream_ptr(qkv.device),
    )
    return q_out


def rope_rows(positions: torch.Tensor, cos: torch.Tensor,
              sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The rotary table rows at each token's position, ``(T, head_dim)`` each: what
    ``quant_linear_rope_append`` reads. Gathered once per forward (one ``edgerag_rope_rows``
    launch), shared by layers. A position outside the table gets a NaN row (its q and k come
    out NaN), as ``rope_append`` does."""
    require_device(positions, cos, sin)
    if positions.dtype != torch.int32 or not positions.is_contiguous():
        raise ValueError("positions must be a contiguous int32 tensor")
    if cos.shape != sin.shape or cos.dim() != 2 or not cos.is_contiguous() or \
            not sin.is_contiguous() or cos.dtype != sin.dtype:
        raise ValueError("cos and sin must be matching contiguous (max_pos, head_dim) tables")
    T = positions.numel()
    c = torch.empty((T, cos.shape[1]), dtype=cos.dtype, device=cos.device)
    s = torch.empty_like(c)
    call("edgerag_rope_rows", positions.data_ptr(), T, cos.data_ptr(), sin.data_ptr(),
         cos.shape[0], cos.shape[1], dtype_code(cos.dtype), c.data_ptr(), s.data_ptr(),
         stream_ptr(positions.device))
    return c, s


def quant_rope_fused(m: int, k: int, bits: int, group_size: int, n_q_heads: int,
                     n_kv_heads: int, head_dim: int, dtype: torch.dtype = torch.float16,
                     normed: bool = False) -> bool:
    """Whether ``quant_linear_rope_append`` runs as one launch (16-byte aligned rows)."""
    return bool(_lib.load().edgerag_quant_linear_rope_append_supported(
        dtype_code(dtype) if dtype in (torch.float16, torch.float32) else -1, m, k, bits,
        group_size, n_q_heads, n_kv_heads, head_dim, int(normed)))


@dataclass
class NormedInput:
    """A projection input ``xw = fp16(w * h)`` written by ``quant_linear_residual`` (w: the norm
    weight, h: the residual stream), plus the producer's per-(token, workgroup) sums of squares of
    h and eps: the projection is then of RMSNorm(h)."""

    partials: torch.Tensor
    n_parts: int
    eps: float

    def args(self, m: int) -> tuple:
        """The C arguments for an m-token input (shapes checked)."""
        if self.partials.dtype != torch.float32 or self.partials.numel() < m * self.n_parts:
            raise ValueError(f"partials must hold {m} x {self.n_parts} float32 sums")
        return (self.partials.data_ptr(), self.n_parts, float(self.eps))


_NO_NORM = (None, 0, 0.0)


def quant_residual_parts(m: int, k: int, n: int, bits: int, group_size: int,
                         dtype: torch.dtype = torch.float16) -> int:
    """Partial sums per token ``quant_linear_residual`` writes for this shape; 0 if not covered."""
    return int(_lib.load().edgerag_quant_linear_residual_parts(
        dtype_code(dtype) if dtype in (torch.float16, torch.float32) else -1, m, k, n, bits,
        group_size))


def quant_linear_residual(
    x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor | None,
    in_features: int, out_features: int, bits: int, group_size: int, hidden: torch.Tensor,
    partials: torch.Tensor, next_norm_weight: torch.Tensor | None = None,
    xw: torch.Tensor | None = None,
) -> int:
    """``hidden += x . W^T`` in place (fp16) plus the per-(token, workgroup) sums of squares of
    the new ``hidden`` rows in ``partials``, and ``xw = fp16(next_norm_weight * hidden)`` when
    given (the input of the next normed projection); returns the sums' count per token. Decode
    batches only (``quant_residual_parts`` > 0): raises otherwise."""
    require_device(x, packed, scales, bias, hidden, partials, next_norm_weight, xw)
    if (next_norm_weight is None) != (xw is None):
        raise ValueError("next_norm_weight and xw go together")
    if xw is not None and (xw.shape != hidden.shape or xw.stride(1) != 1 or
                           xw.dtype != torch.float16 or next_norm_weight.shape != (out_features,)
                           or next_norm_weight.dtype != torch.float16):
        raise ValueError("xw must match hidden; next_norm_weight must be fp16 (out_features,)")
    x2 = x.reshape(-1, in_features)
    if x2.stride(1) != 1 or (x2.stride(0) * x2.element_size()) % 16 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    if hidden.shape != (m, out_features) or hidden.stride(1) != 1 or hidden.dtype != torch.float16:
        raise ValueError(f"hidden must be fp16 ({m}, {out_features}) with contiguous rows")
    if partials.dtype != torch.float32 or not partials.is_contiguous():
        raise ValueError("partials must be a contiguous float32 tensor")
    if scales.dtype != torch.float16:
        scales = scales.to(torch.float16)
    n_parts = ctypes.c_int32(0)
    call(
        "edgerag_quant_linear_residual", x2.data_ptr(), dtype_code(x2.dtype), x2.stride(0), m,
        in_features, packed.data_ptr(), scales.contiguous().data_ptr(), ptr(bias), out_features,
        bits, group_size, hidden.data_ptr(), hidden.stride(0), partials.data_ptr(),
        partials.numel(), ctypes.addressof(n_parts), ptr(next_norm_weight), ptr(xw),
        xw.stride(0) if xw is not None else 0, stream_ptr(x.device),
    )
    return int(n_parts.value)


def quant_linear_rope_append(
    x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor | None,
    in_features: int, bits: int, group_size: int, positions: torch.Tensor, cos: torch.Tensor,
    sin: torch.Tensor, n_q_heads: int, n_kv_heads: int, head_dim: int, slots: torch.Tensor,
    key_pool: torch.Tensor, value_pool: torch.Tensor, q_out: torch.Tensor | None = None,
    rows: tuple[torch.Tensor, torch.Tensor] | None = None, norm: NormedInput | None = None,
) -> torch.Tensor:
    """The fused q/k/v quant linear, RoPE and KV append; returns q ``(T, n_q_heads, head_dim)``.

    One launch where the native library covers the shape and ``rows`` (``rope_rows`` of the
    step) is given; otherwise ``quant_linear`` then ``rope_append``. Both give the same bits.
    ``norm``: x is a residual producer's ``xw`` and the projection is of RMSNorm of its residual
    stream (one launch only)."""
    require_device(x, packed, scales, bias, positions, cos, sin, slots, key_pool, value_pool,
                   q_out)
    n = (n_q_heads + 2 * n_kv_heads) * head_dim
    x2 = x.reshape(-1, in_features)
    if x2.stride(1) != 1 or (x2.stride(0) * x2.element_size()) % 16 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    T = x2.shape[0]
    if q_out is None:
        q_out = torch.empty((T, n_q_heads, head_dim), dtype=x.dtype, device=x.device)
    fused = (
        rows is not None and T > 0 and x2.dtype == torch.float16 and packed.data_ptr() % 16 == 0
        and key_pool.dtype == torch.float16 and slots.dtype == torch.int32
        and quant_rope_fused(T, in_features, bits, group_size, n_q_heads, n_kv_heads, head_dim,
                             normed=norm is not None)
    )
    if norm is not None and not fused:
        raise ValueError("a normed input needs the one-launch path (decode batch, rope rows)")
    if not fused:
        qkv = quant_linear(x2, packed, scales, bias, in_features, n, bits, group_size,
                           split_k=False)
        return rope_append(qkv, positions, cos, sin, n_q_heads, n_kv_heads, head_dim, slots,
                           key_pool, value_pool, q_out=q_out)
    _check_pool(key_pool, "key_pool")
    _check_pool(value_pool, "value_pool")
    nkv, num_blocks, block_size, d = key_pool.shape
    if (nkv, d) != (n_kv_heads, head_dim) or value_pool.shape != key_pool.shape:
        raise ValueError("pools do not match the heads")
    cos_tok, sin_tok = rows
    if cos_tok.shape != (T, head_dim) or sin_tok.shape != (T, head_dim) or \
            cos_tok.dtype != torch.float16 or not (cos_tok.is_contiguous() and sin_tok.is_contiguous()):
        raise ValueError(f"rope rows must be contiguous fp16 ({T}, {head_dim})")
    if q_out.shape != (T, n_q_heads, head_dim) or q_out.stride(2) != 1 or \
            q_out.stride(1) != head_dim:
        raise ValueError("q_out must be (tokens, n_q_heads, head_dim) with packed heads")
    if scales.dtype != torch.float16:
        scales = scales.to(torch.float16)
    if bias is not None and bias.dtype != torch.float16:
        bias = bias.to(torch.float16)
    call(
        "edgerag_quant_linear_rope_append", x2.data_ptr(), dtype_code(x2.dtype), x2.stride(0), T,
        in_features, packed.data_ptr(), scales.contiguous().data_ptr(), ptr(bias), bits,
        group_size, cos_tok.data_ptr(), sin_tok.data_ptr(), n_q_heads, n_kv_heads, head_dim,
        q_out.data_ptr(), q_out.stride(0), slots.data_ptr(), key_pool.data_ptr(),
        value_pool.data_ptr(), num_blocks, block_size,
        *(norm.args(T) if norm is not None else _NO_NORM), stream_ptr(x.device),
    )
    return q_out


def silu_mul(gate_up: torch.Tensor, intermediate: int,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """SwiGLU activation of the fused ``[gate | up]`` rows: ``(T, 2I) -> (T, I)``."""
    require_device(gate_up, out)
    T = gate_up.shape[0]
    if gate_up.dim() != 2 or gate_up.stride(1) != 1 or gate_up.shape[1] != 2 * intermediate:
        raise ValueError("gate_up must be (tokens, 2 * intermediate) with contiguous rows")
    if out is None:
        out = torch.empty((T, intermediate), dtype=gate_up.dtype, device=gate_up.device)
    call("edgerag_silu_mul", gate_up.data_ptr(), gate_up.stride(0), T, intermediate,
         out.data_ptr(), out.stride(0), dtype_code(gate_up.dtype), stream_ptr(gate_up.device))
    return out


def quant_swiglu_fused(m: int, k: int, n: int, bits: int, group_size: int,
                       dtype: torch.dtype = torch.float16, normed: bool = False) -> bool:
    """Whether ``quant_linear_swiglu`` runs as one launch for this shape (16-byte aligned rows)."""
    return bool(_lib.load().edgerag_quant_linear_swiglu_supported(
        dtype_code(dtype) if dtype in (torch.float16, torch.float32) else -1, m, k, n, bits,
        group_size, int(normed)))


def quant_linear_swiglu(
    x: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    bias: torch.Tensor | None,
    in_features: int,
    out_features: int,
    bits: int,
    group_size: int,
    out: torch.Tensor | None = None,
    norm: NormedInput | None = None,
) -> torch.Tensor:
    """SwiGLU of the fused ``[gate; up]`` quant linear: ``x (T, K) -> (T, out_features / 2)``.

    One launch where the native library covers the shape (decode batches of INT8 per-channel
    weights); otherwise the projection and ``silu_mul`` as two launches. Both give the same bits.
    ``norm``: x is a residual producer's ``xw`` and the projection is of RMSNorm of its residual
    stream (one launch only).
    """
    require_device(x, packed, scales, bias, out)
    inter = out_features // 2
    if out_features % 2:
        raise ValueError("a fused [gate; up] weight has an even number of rows")
    x2 = x.reshape(-1, in_features)
    if x2.stride(1) != 1 or (x2.stride(0) * x2.element_size()) % 16 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    fused = not (m == 0 or x2.dtype != torch.float16 or packed.data_ptr() % 16
                 or not quant_swiglu_fused(m, in_features, out_features, bits, group_size,
                                           normed=norm is not None))
    if norm is not None and not fused:
        raise ValueError("a normed input needs the one-launch path (decode batch)")
    if not fused:
        gu = quant_linear(x2, packed, scales, bias, in_features, out_features, bits, group_size,
                          split_k=False)
        return silu_mul(gu, inter, out=out)
    y = out if out is not None else torch.empty((m, inter), dtype=x.dtype, device=x.device)
    if y.shape != (m, inter) or y.stride(1) != 1:
        raise ValueError(f"out must be ({m}, {inter}) with contiguous rows")
    if scales.dtype != torch.float16:
        scales = scales.to(torch.float16)
    if bias is not None and bias.dtype != torch.float16:
        bias = bias.to(torch.float16)
    call(
        "edgerag_quant_linear_swiglu", x2.data_ptr(), dtype_code(x2.dtype), x2.stride(0), m,
        in_features, packed.data_ptr(), scales.contiguous().data_ptr(), ptr(bias), out_features,
        bits, group_size, y.data_ptr(), y.stride(0),
        *(norm.args(m) if norm is not None else _NO_NORM), stream_ptr(x.device),
    )
    return y


# --- quantisation -----------------------------------------------------------------------------


def quantize(weight: torch.Tensor, bits: int, group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``(packed uint8, scales fp16)`` for ``weight (N, K)``; bit-identical to the reference."""
    require_device(weight)
    if weight.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(weight.shape)}")
    weight = weight.contiguous()
    n, k = weight.shape
    width = k // 2 if bits == 4 else k
    packed = torch.empty((n, width), dtype=torch.uint8, device=weight.device)
    scales = torch.empty((n, max(k // group_size, 0)), dtype=torch.float16, device=weight.device)
    call(
        "edgerag_quantize", weight.data_ptr(), dtype_code(weight.dtype), n, k, bits, group_size,
        packed.data_ptr(), scales.data_ptr(), stream_ptr(weight.device),
    )
    return packed, scales


def argmax_rows(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """int32 ``(rows,)``: the first index of each row's maximum (a NaN counts as the maximum),
    like ``x.argmax(dim=-1)``; one launch (the executor's greedy token choice)."""
    require_device(x, out)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("argmax_rows takes (rows, cols) with contiguous rows")
    rows, cols = x.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.int32, device=x.device)
    call("edgerag_argmax_rows", x.data_ptr(), dtype_code(x.dtype), rows, cols, x.stride(0),
         out.data_ptr(), stream_ptr(x.device))
    return out


LM_HEAD_MAX_ROWS = 16
_LM_WORKSPACES: dict[tuple[torch.device, int], torch.Tensor] = {}


def lm_head_fused(x: torch.Tensor) -> bool:
    """Whether ``lm_head_argmax`` takes the hidden rows ``x (m, k)``: fp16, 1..16 rows of a width
    the kernel stages, 16-byte aligned rows."""
    m, k = x.shape
    return (x.dtype == torch.float16 and x.stride(1) == 1 and (x.stride(0) * 2) % 16 == 0
            and x.data_ptr() % 16 == 0
            and bool(_lib.load().edgerag_lm_head_argmax_supported(m, k)))


def lm_head_argmax(x: torch.Tensor, weight: torch.Tensor, logits: torch.Tensor | None = None,
                   tokens: torch.Tensor | None = None) -> tuple[torch.Tensor | None, torch.Tensor]:
    """``logits = x @ weight.T`` (fp16, written into ``logits`` when given) and each row's
    greedy token (int32, ``tokens``), for up to 16 rows, in two launches; the weight streams from
    HBM once. The candidate workspace is allocated once per (device, vocabulary) and reused, so a
    graph that captured the call keeps a valid address."""
    require_device(x, weight, logits, tokens)
    m, k = x.shape
    vocab = weight.shape[0]
    if not 1 <= m <= LM_HEAD_MAX_ROWS:
        raise ValueError(f"lm_head_argmax takes 1..{LM_HEAD_MAX_ROWS} rows, got {m}")
    if x.dtype != torch.float16 or weight.dtype != torch.float16 or weight.shape[1] != k:
        raise ValueError("lm_head_argmax takes fp16 x (m, k) and weight (vocab, k)")
    if x.stride(1) != 1 or not weight.is_contiguous():
        raise ValueError("x rows and the weight must be contiguous")
    if tokens is None:
        tokens = torch.empty(m, dtype=torch.int32, device=x.device)
    if logits is not None and (logits.shape != (m, vocab) or logits.dtype != torch.float16
                               or logits.stride(1) != 1):
        raise ValueError(f"logits must be fp16 ({m}, {vocab}) with contiguous rows")
    key = (x.device, vocab)
    ws = _LM_WORKSPACES.get(key)
    if ws is None:
        nbytes = int(_lib.load().edgerag_lm_head_workspace_bytes(LM_HEAD_MAX_ROWS, vocab))
        ws = _LM_WORKSPACES[key] = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    call("edgerag_lm_head_argmax", x.data_ptr(), x.stride(0), m, k, weight.data_ptr(), vocab,
         ptr(logits), 0 if logits is None else logits.stride(0), tokens.data_ptr(),
         ws.data_ptr(), ws.numel(), stream_ptr(x.device))
    return logits, tokens


def dequantize(packed: torch.Tensor, scales: torch.Tensor, in_features: int, bits: int,
               group_size: int) -> torch.Tensor:
    """fp16 ``(N, K)`` weight rebuilt from codes and scales, as the reference dequantizes."""
    require_device(packed, scales)
    n = packed.shape[0]
    out = torch.empty((n, in_features), dtype=torch.float16, device=packed.device)
    scales = scales.to(torch.float16).contiguous()
    call(
        "edgerag_dequantize", packed.contiguous().data_ptr(), scales.data_ptr(), n, in_features,
        bits, group_size, out.data_ptr(), stream_ptr(packed.device),
    )
    return out


def quant_linear(
    x: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    bias: torch.Tensor | None,
    in_features: int,
    out_features: int,
    bits: int,
    group_size: int,
    out: torch.Tensor | None = None,
    split_k: bool = True,
) -> torch.Tensor:
    """``x (..., K) -> (..., N)`` through the fused dequant + GEMV/GEMM kernels.

    ``split_k``: shapes whose tile grid would leave CUs idle split K over the per-device
    workspace (``edgerag_quant_linear_ws``); False runs ``edgerag_quant_linear``, whose bits the
    fused-epilogue launches reproduce exactly."""
    require_device(x, packed, scales, bias)
    if x.shape[-1] != in_features:
        raise ValueError(f"input has {x.shape[-1]} features, layer expects {in_features}")
    if x.dtype not in (torch.float16, torch.float32):
        raise TypeError(f"quant_linear takes float16 or float32 activations, not {x.dtype}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, in_features)
    if x2.stride(1) != 1 or (x2.stride(0) * x2.element_size()) % 16 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    if out is None:
        y = torch.empty((m, out_features), dtype=x.dtype, device=x.device)
    else:
        y = out.view(m, out_features)
    if scales.dtype != torch.float16:
        scales = scales.to(torch.float16)
    if bias is not None and bias.dtype != torch.float16:
        bias = bias.to(torch.float16)
    args = (x2.data_ptr(), dtype_code(x2.dtype), x2.stride(0), m, in_features, packed.data_ptr(),
            scales.contiguous().data_ptr(), ptr(bias), out_features, bits, group_size,
            y.data_ptr(), y.stride(0))
    if split_k:
        ws = quant_workspace(x.device)
        call("edgerag_quant_linear_ws", *args, ws.data_ptr(), ws.numel(), stream_ptr(x.device))
    else:
        call("edgerag_quant_linear", *args, stream_ptr(x.device))
    return y.view(*lead, out_features)
