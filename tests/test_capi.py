"""The C ABI: the library loads, exports every declared symbol, and its host-only planner is
correct. No GPU is touched: only entry points that validate and return before any HIP call run.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from edgerag_amd import _lib, kernels

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def declared_symbols() -> set[str]:
    names: set[str] = set()
    for header in HEADERS:
        text = header.read_text()
        names |= set(re.findall(r"^(?:int64_t|int|const char\*)\s+(edgerag_\w+)\s*\(", text,
                                flags=re.M))
    return names


def test_library_exports_every_declared_symbol() -> None:
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert names == set(_lib.SIGNATURES), "ctypes signatures and header diverged"
    assert _lib.version().startswith("edgerag_amd")


def test_measurement_probes_live_in_a_bench_only_library() -> None:
    """The product library exports no probe; the probe library exports its header's symbols."""
    from edgerag_amd._build import PROBE_LIB_PATH

    lib = _lib.load()
    assert not hasattr(lib, "edgerag_probe_read") and not hasattr(lib, "edgerag_probe_gather")
    header = Path(__file__).resolve().parents[1] / "edgerag_amd/csrc/probe/edgerag_probe.h"
    probe_names = set(re.findall(r"^int\s+(edgerag_probe_\w+)\s*\(", header.read_text(),
                                 flags=re.M))
    assert probe_names == {"edgerag_probe_read", "edgerag_probe_gather"}
    probe = ctypes.CDLL(str(PROBE_LIB_PATH))
    assert all(hasattr(probe, n) for n in probe_names)


def test_swiglu_support_query() -> None:
    """The fused SwiGLU linear covers decode batches of wide INT8 per-channel [gate; up]
    weights (normed inputs up to 16 tokens) and prefill slices whose plain launch takes 128-row
    weight tiles; the query answers without touching a GPU."""
    q = _lib.load().edgerag_quant_linear_swiglu_supported
    F16, F32 = 1, 0
    assert q(F16, 8, 2048, 16384, 8, 2048, 0) == 1  # config 5's gate/up, a decode batch
    assert q(F16, 8, 2048, 16384, 8, 2048, 1) == 1  # ... with the RMSNorm folded in
    assert q(F16, 64, 2048, 16384, 8, 2048, 0) == 1
    assert q(F16, 17, 2048, 16384, 8, 2048, 1) == 0  # normed: at most 16 tokens
    assert q(F16, 65, 2048, 16384, 8, 2048, 0) == 1  # prefill slices: the tiled GEMM
    assert q(F16, 519, 2048, 16384, 8, 2048, 0) == 1  # a chunk + 7 decode rows
    assert q(F16, 65, 2048, 16384, 8, 2048, 1) == 0  # normed: at most 16 tokens
    assert q(F16, 80, 1024, 2048, 8, 1024, 0) == 0  # 64x64 tiles: gate and up in other waves
    assert q(F16, 0, 2048, 16384, 8, 2048, 0) == 0
    assert q(F16, 8, 2048, 4096, 8, 2048, 0) == 0  # one 16-row tile per workgroup
    assert q(F16, 8, 2048, 16383, 8, 2048, 0) == 0  # odd N: no [gate; up] split
    assert q(F16, 8, 2048, 16384, 4, 128, 0) == 0  # INT4
    assert q(F16, 8, 2048, 16384, 8, 128, 0) == 0  # grouped INT8
    assert q(F32, 8, 2048, 16384, 8, 2048, 0) == 0
    assert q(F16, 8, 200, 16384, 8, 200, 0) == 0  # K not a multiple of 64


def test_quant_workspace_query() -> None:
    """The workspace route is planned on the host. For decode batches past the streaming GEMV's
    crossover, and for larger M whose 64x64 tile grid leaves CUs idle, the tiled GEMM splits K
    where its cost model (a fixed 12 steps for the partials' round trip, plus 64-k steps per
    split times rounds of workgroups over the 256 CUs) says so; the workspace holds the fp32
    partial tiles."""
    q = kernels.quant_workspace_bytes
    tile = 64 * 64 * 4
    assert q(64, 8192, 2048, 8, 8192) == 32 * 8 * tile  # 32 tiles x 8 splits: 12 + 16 steps
    assert q(64, 2048, 2048, 8, 2048) == 32 * 8 * tile  # 12 + 4 steps, against 32
    assert q(128, 2048, 2048, 8, 2048) == 64 * 4 * tile  # 64 tiles x 4
    assert q(64, 2048, 8192, 8, 2048) == 128 * 2 * tile  # 128 tiles: 12 + 16 steps beat 32
    assert q(40, 1152, 4608, 4, 128) == 0  # INT4: 18 steps, too few to pay for a split
    assert q(24, 8192, 2048, 8, 8192) == 32 * 8 * tile  # K >= 4096: from 17 tokens
    assert q(32, 2048, 2048, 8, 2048) == 0  # below 40 tokens on small layers: streaming GEMV
    assert q(48, 2048, 2048, 8, 2048) == 0  # 4M codes: from 64 tokens
    assert q(64, 1152, 1152, 4, 128) == 0  # 1.3M codes: the skinny GEMV at every batch size
    assert q(16, 8192, 2048, 8, 8192) == 0
    assert q(512, 2048, 8192, 8, 2048) == 0  # 128x64 tiles fill the GPU: the plain launch
    assert q(64, 128, 2048, 8, 128) == 0  # two 64-k steps: nothing to split
    assert q(64, 2048, 2048, 8, 48) == 0  # group not a multiple of 32
    # 96 tiles: 8 splits would model cheaper but need 12 MiB of partials; the bound keeps 2.
    assert q(64, 2048, 6144, 8, 2048) == 96 * 2 * tile
    for m in (17, 24, 40, 64, 100, 200, 300):
        for k, n in [(8192, 2048), (2048, 6144), (2048, 16384), (8192, 64), (1152, 37), (2048, 4100)]:
            assert 0 <= q(m, k, n, 8, k) <= _lib.QUANT_WORKSPACE_MAX, (m, k, n)


def test_rope_append_support_query() -> None:
    """The fused q/k/v + RoPE + KV append covers decode batches whose plain projection launch
    streams with one k-slice; the query answers without touching a GPU."""
    q = _lib.load().edgerag_quant_linear_rope_append_supported
    F16 = 1
    assert q(F16, 8, 2048, 8, 2048, 32, 32, 64, 0) == 1  # config 5's q/k/v, a decode batch
    assert q(F16, 8, 2048, 8, 2048, 32, 32, 64, 1) == 1  # ... with the RMSNorm folded in
    assert q(F16, 20, 2048, 8, 2048, 32, 32, 64, 1) == 0  # normed: at most 16 tokens
    assert q(F16, 64, 2048, 8, 2048, 32, 8, 64, 0) == 1  # GQA, N 3072: one k-slice from M > 32
    # Two k-slices (N 3072 at M <= 32; N 6144 at M <= 8): 8-row tiles pairing rotate_half twins.
    assert q(F16, 8, 2048, 8, 2048, 32, 8, 64, 0) == 1
    assert q(F16, 24, 2048, 8, 2048, 32, 8, 64, 0) == 1
    assert q(F16, 8, 16384, 8, 16384, 32, 32, 64, 0) == 1
    # N 4096 (256 one-slice workgroups, evenly spread): one k-slice, 16 waves at K 16384.
    assert q(F16, 8, 16384, 8, 16384, 32, 16, 64, 0) == 0
    assert q(F16, 65, 2048, 8, 2048, 32, 32, 64, 0) == 0
    assert q(F16, 8, 2048, 8, 2048, 32, 32, 48, 0) == 0  # head_dim not a multiple of 32
    assert q(F16, 8, 2048, 4, 128, 32, 32, 64, 0) == 0  # INT4
    assert q(0, 8, 2048, 8, 2048, 32, 32, 64, 0) == 0  # fp32 activations


def test_lm_head_support_query() -> None:
    """The fused lm_head + argmax stages m rows of width k in 128 KiB of LDS; wider batches (such
    as 16 rows of a 4,096-wide model: 131,328 bytes) are declined beforehand, so the decoder takes
    the vendor GEMM + argmax path instead of failing the step."""
    q = _lib.load().edgerag_lm_head_argmax_supported
    assert q(1, 2048) == 1 and q(16, 2048) == 1  # config 5
    assert q(16, 4096) == 0 and q(15, 4096) == 1  # 15 * 513 * 16 = 123,120 bytes
    assert q(1, 8160) == 1 and q(17, 2048) == 0 and q(0, 2048) == 0
    assert q(4, 2000) == 0 and q(4, 16) == 0  # k a multiple of 32, at least 32


def test_residual_parts_query() -> None:
    """The residual-add producer covers decode batches (up to 16 tokens) of the streaming
    shapes and reports how many partial sums per token it writes: one per workgroup."""
    q = _lib.load().edgerag_quant_linear_residual_parts
    F16 = 1
    assert q(F16, 8, 2048, 2048, 8, 2048) == 256  # o_proj: 8-row tiles (two k-slices)
    assert q(F16, 8, 8192, 2048, 8, 8192) == 256  # down_proj
    assert q(F16, 1, 2048, 4096, 8, 2048) == 256  # 16-row tiles
    assert q(F16, 16, 2048, 8192, 8, 2048) == 256  # two 16-row tiles per workgroup
    assert q(F16, 17, 2048, 2048, 8, 2048) == 0  # more than 16 tokens
    assert q(F16, 8, 2048, 2048, 4, 128) == 0  # INT4
    assert q(0, 8, 2048, 2048, 8, 2048) == 0


def test_validation_errors_come_back_as_messages() -> None:
    with pytest.raises(_lib.EdgeragError, match="only 4- and 8-bit"):
        _lib.call("edgerag_quant_linear", None, 1, 16, 1, 16, None, None, None, 4, 3, 16, None,
                  4, None)
    with pytest.raises(_lib.EdgeragError, match="not divisible by group_size"):
        _lib.call("edgerag_quantize", None, 1, 4, 100, 4, 128, None, None, None)
    with pytest.raises(_lib.EdgeragError, match="pool dims"):
        _lib.call("edgerag_kv_append", None, None, 1, 0, 0, None, 1, None, None, 1, 0, 1, 16,
                  64, None)
    with pytest.raises(_lib.EdgeragError, match="not a plan"):
        _lib.call(
            "edgerag_paged_attention",
            None, None, 0,          # plan_host, plan_dev, plan_words
            None, 0, 0,             # q, strides
            None, None, 1,          # pools, dtype
            None, 0, None, None,    # block tables, stride, query_start_loc, context_lens
            0, 0, 4, 4, 64, 16, 1,  # num_reqs, num_tokens, heads, head_dim, block, num_blocks
            1.0, None, 0, 0,        # scale, out, strides
            None, 0, 7, None,       # workspace, bytes, parts (all), stream
        )
    for parts in (8, 16, 0):  # the shared modifier alone, an unknown bit, nothing
        with pytest.raises(_lib.EdgeragError, match="parts mask"):
            _lib.call("edgerag_paged_attention", None, None, 0, None, 0, 0, None, None, 1, None,
                      0, None, None, 0, 0, 4, 4, 64, 16, 1, 1.0, None, 0, 0, None, 0, parts, None)
    with pytest.raises(_lib.EdgeragError, match="capacities"):
        _lib.call("edgerag_paged_attention_fixed", 16, -1, 0, 1, 0, 0, 0, 16, 0, 0, 16, 16, 1,
                  16, 0, 16, 16, 4, 4, 64, 16, 1, 1.0, 16, 0, 0, None, 0, None)
    with pytest.raises(_lib.EdgeragError, match="row_waves"):  # past the 16-wave merge space
        _lib.call("edgerag_paged_attention_fixed", 16, 4, 0, 1, 0, 17, 0, 16, 0, 0, 16, 16, 1,
                  16, 0, 16, 16, 4, 4, 64, 16, 1, 1.0, 16, 0, 0, None, 0, None)
    with pytest.raises(_lib.EdgeragError, match="row_waves"):  # head_dim past 128
        _lib.call("edgerag_paged_attention_fixed", 16, 4, 0, 1, 0, 16, 0, 16, 0, 0, 16, 16, 1,
                  16, 0, 16, 16, 4, 4, 256, 16, 1, 1.0, 16, 0, 0, None, 0, None)
    # Slots: past 32, without workgroup rows, or more than the partials hold (2 rows x 4 heads x
    # 16 slots = 128 > 100).
    for rows, partials, row_waves, slots in ((2, 4096, 8, 64), (2, 4096, 0, 16),
                                             (2, 100, 8, 16)):
        with pytest.raises(_lib.EdgeragError, match="slots"):
            _lib.call("edgerag_paged_attention_fixed", 16, 4, rows, 1, partials, row_waves,
                      slots, 16, 0, 0, 16, 16, 1, 16, 0, 16, 16, 4, 4, 64, 16, 1, 1.0, 16, 0, 0,
                      16, 1 << 20, None)
    with pytest.raises(_lib.EdgeragError, match="width"):
        _lib.call("edgerag_rmsnorm", None, 0, None, 0, None, None, 0, None, 0, 1, 0, 1e-5, 1,
                  None)
    with pytest.raises(_lib.EdgeragError, match="bad shape"):
        _lib.call("edgerag_rope_append", None, 0, None, None, None, 8, 1, 4, 4, 63, None, 0, None,
                  None, None, 1, 16, 1, None)
    with pytest.raises(_lib.EdgeragError, match="bad shape"):
        _lib.call("edgerag_silu_mul", None, 0, 1, 0, None, 0, 1, None)
    # The tiled q/k/v + RoPE launch (M = 512, 32 + 2 x 32 heads of 64) reads cos / sin rows in
    # 8-byte runs: a table 2 bytes off is refused before anything is launched.
    base = 1 << 20
    with pytest.raises(_lib.EdgeragError, match="8-byte aligned"):
        _lib.call("edgerag_quant_linear_rope_append", base, 1, 2048, 512, 2048, base, base, None,
                  8, 2048, base + 2, base, 32, 32, 64, base, 2048, base, base, base, 16, 16,
                  None, 0, 1e-5, None)


def test_device_guard_refuses_cpu_tensors() -> None:
    with pytest.raises(ValueError, match="MI355X only"):
        kernels.kv_gather(torch.zeros(1, 1, 16, 8), torch.zeros(1, dtype=torch.int32), 1)


# --- the host planner ---------------------------------------------------------------------------

ITEM_WORDS, REQ_WORDS = 8, 4


def decode_plan(plan: np.ndarray):
    n_items, n_reqs, item_off, req_off = (int(plan[i]) for i in (2, 3, 4, 5))
    items = plan[item_off : item_off + n_items * ITEM_WORDS].reshape(n_items, ITEM_WORDS)
    reqs = plan[req_off : req_off + n_reqs * REQ_WORDS].reshape(n_reqs, REQ_WORDS)
    return items, reqs


def check_coverage(qsl, ctx, n_q, n_kv, bs=16):
    """Every (token, q-head, visible key) is covered by exactly one (item, split)."""
    plan, ws = kernels.make_plan_host(np.array(qsl, np.int32), np.array(ctx, np.int32), n_q, n_kv,
                                      64, bs, max(1, -(-max(ctx + [1]) // bs)), torch.float16)
    items, reqs = decode_plan(plan)
    n_rep = n_q // n_kv
    seen: dict[tuple[int, int, int], int] = {}
    for r, h, qb, qc, kb, ke, split, _kind in items.tolist():
        q0, c, L = qsl[r], qsl[r + 1] - qsl[r], ctx[r]
        assert q0 <= qb and qb + qc <= q0 + c
        nsplit, split_len = reqs[r][0], reqs[r][1]
        assert kb == split * split_len and ke <= min(L, (split + 1) * split_len)
        for t in range(qb, qb + qc):
            lim = L - c + (t - q0)
            for hq in range(h * n_rep, (h + 1) * n_rep):
                key = (t, hq, split)
                assert key not in seen
                seen[key] = min(ke, lim + 1) - kb
    n_partials = 0
    slots = int(plan[21])
    for r in range(len(ctx)):
        q0, c, L = qsl[r], qsl[r + 1] - qsl[r], ctx[r]
        nsplit, split_len, part_off, pstride = (int(w) for w in reqs[r])
        row = c * n_rep <= 8
        # Slotted row requests: S slots per (token, head), even when not split.
        assert pstride == (slots if slots and row else nsplit), r
        assert nsplit <= pstride
        assert part_off == n_partials, r
        if c and (nsplit > 1 or (slots and row)):
            n_partials += c * n_q * pstride
        for t in range(q0, q0 + c):
            lim = L - c + (t - q0)
            for hq in range(n_q):
                covered = sum(max(0, seen.get((t, hq, s), 0)) for s in range(max(nsplit, 0)))
                assert covered == lim + 1, (r, t, hq)
    assert int(plan[6]) == n_partials
    if n_partials == 0:
        assert ws == 0
    return items


def check_parts(ctx, h, bs, items, reqs, plan) -> None:
    """A batch of fewer row workgroups than CUs: each context in equal whole-block parts of at
    least 8 waves x 32 tokens (x 16 when no context passes 2,048 tokens), about 512 workgroups in
    all (never more than 512 plus one per request and head), their partials in fixed slots: every
    token has a merge row."""
    work = sum(ctx) * h
    wave_tokens = -(-(16 if max(ctx) <= 2048 else 32) // bs) * bs
    part = min(8 * 64 * bs, max(8 * wave_tokens, -(-(-(-work // 512)) // bs) * bs))
    slots = int(plan[21])
    if max(ctx) <= part:  # no context cut: nothing to merge, no slots
        assert slots == 0 and int(plan[16]) == 0
        return
    part = max(part, -(-(-(-max(ctx) // slots)) // bs) * bs)  # at most `slots` parts
    for r, L in enumerate(ctx):
        n = -(-L // part) if L > part else 1
        slen = max(L, 1) if n == 1 else -(-(-(-L // n)) // bs) * bs
        assert (int(reqs[r][0]), int(reqs[r][1])) == (-(-L // slen) if L else 0, slen), r
    assert items.shape[0] <= 512 + len(ctx) * h
    # Parts in fixed slots: a power of two covering 512 / h parts (at most 32); every token of the
    # batch has a merge row, in token order, naming its slots.
    assert slots == min(32, 1 << max(1, (-(-512 // h) - 1).bit_length()))
    assert all(int(reqs[r][0]) <= slots for r in range(len(ctx)))
    n_tok = len(ctx)
    assert int(plan[16]) == n_tok
    comb = plan[int(plan[17]) : int(plan[17]) + 8 * n_tok].reshape(n_tok, 8)
    for t, e in enumerate(comb.tolist()):
        assert e[0] == t and e[6] == t * h * slots and e[7] == slots, e


def test_fixed_capacity_bounds_the_planner() -> None:
    """edgerag_attn_fixed_row_items bounds the row items of every decode-only plan with
    workgroup rows, across batch sizes and context lengths."""
    q = _lib.load().edgerag_attn_fixed_row_items
    rng = np.random.default_rng(5)
    for cap in (1, 2, 4, 8):
        bound = q(cap, 32, 8192, 16)
        assert bound >= 512
        for _ in range(60):
            n = int(rng.integers(1, cap + 1))
            ctx = rng.integers(1, 8193, n).astype(np.int32)
            plan, _ = kernels.make_plan_host(np.arange(n + 1, dtype=np.int32), ctx, 32, 32, 64,
                                             16, 512, torch.float16)
            if int(plan[19]):
                assert int(plan[13]) <= bound, (cap, ctx.tolist())
    assert q(-1, 32, 8192, 16) == -1


@given(
    reqs=st.lists(
        st.tuples(st.integers(0, 3000), st.integers(0, 600)), min_size=1, max_size=12
    ),
    heads=st.sampled_from([(4, 4), (9, 3), (8, 2), (32, 32)]),
)
@settings(max_examples=40, deadline=None)
def test_plan_covers_every_visible_key_exactly_once(reqs, heads) -> None:
    ctx, q_lens = [], []
    for L, c in reqs:
        c = min(c, L)
        ctx.append(L)
        q_lens.append(c)
    qsl = [0]
    for c in q_lens:
        qsl.append(qsl[-1] + c)
    check_coverage(qsl, ctx, *heads)


def test_plan_for_cfg1_and_ordering() -> None:
    items = check_coverage([0, 1, 2, 3, 4], [37, 128, 300, 511], 9, 3)
    costs = (items[:, 5] - items[:, 4]).tolist()
    assert costs == sorted(costs, reverse=True), "items must be heaviest first"


def test_plan_rejects_bad_batches() -> None:
    with pytest.raises(_lib.EdgeragError, match="queries but context"):
        kernels.make_plan_host(np.array([0, 5], np.int32), np.array([4], np.int32), 4, 4, 64, 16,
                               8, torch.float16)
    with pytest.raises(_lib.EdgeragError, match="block table holds"):
        kernels.make_plan_host(np.array([0, 1], np.int32), np.array([100], np.int32), 4, 4, 64,
                               16, 2, torch.float16)
    with pytest.raises(_lib.EdgeragError, match="query heads against"):
        kernels.make_plan_host(np.array([0, 1], np.int32), np.array([10], np.int32), 6, 4, 64, 16,
                               2, torch.float16)
    with pytest.raises(_lib.EdgeragError, match="head_dim"):
        kernels.make_plan_host(np.array([0, 1], np.int32), np.array([10], np.int32), 4, 4, 48, 16,
                               2, torch.float16)


def test_plan_size_query_without_buffer() -> None:
    words, ws = ctypes.c_int64(0), ctypes.c_int64(0)
    qsl = np.arange(9, dtype=np.int32)
    ctx = np.full(8, 4000, np.int32)
    _lib.call("edgerag_attn_plan", qsl.ctypes.data, ctx.ctypes.data, 8, 32, 32, 64, 16, 400, 1,
              None, 0, ctypes.byref(words), ctypes.byref(ws))
    assert words.value > 16 and ws.value == 0  # a workgroup per (request, head): no partials
    _lib.call("edgerag_attn_plan_ex", qsl.ctypes.data, ctx.ctypes.data, 8, 32, 32, 64, 16, 400, 1,
              _lib.PLAN_SPLIT_ROWS, None, 0, ctypes.byref(words), ctypes.byref(ws))
    assert words.value > 16 and ws.value > 0  # KV splits: fp32 partials
    qsl = np.array([0, 1], np.int32)
    ctx = np.array([4000], np.int32)
    _lib.call("edgerag_attn_plan", qsl.ctypes.data, ctx.ctypes.data, 1, 32, 32, 64, 16, 400, 1,
              None, 0, ctypes.byref(words), ctypes.byref(ws))
    assert ws.value > 0  # one request: its context cut into parts, merged through partials
    ctx = np.array([5000], np.int32)
    _lib.call("edgerag_attn_plan", qsl.ctypes.data, ctx.ctypes.data, 1, 32, 32, 64, 16, 400, 1,
              None, 0, ctypes.byref(words), ctypes.byref(ws))
    assert ws.value > 0  # a long context keeps KV splits
    small = np.empty(4, np.int32)
    with pytest.raises(_lib.EdgeragError, match="capacity"):
        _lib.call("edgerag_attn_plan", qsl.ctypes.data, ctx.ctypes.data, 1, 32, 32, 64, 16, 400,
                  1, small.ctypes.data, 4, ctypes.byref(words), ctypes.byref(ws))


@pytest.mark.parametrize(
    "ctx,d,bs,split_rows,row_waves,row_waves_tiles",
    [
        # Fewer than 256 row workgroups (32 kv heads x 3 requests): workgroups of 8 waves over
        # parts of the contexts, whatever their length.
        ([4096, 1, 300], 64, 16, False, 8, 8),
        ([4097, 1, 300], 64, 16, False, 8, 8),
        ([8000], 64, 16, False, 8, 8),
        # 256 row workgroups: one per (request, head) when every context fits 16 waves x 256
        # tokens; else KV splits, but beside prefill tiles workgroup rows (parts of up to 512
        # tokens per wave) once their 32 kv heads x 8 requests cover the 256 CUs.
        ([4096] + [300] * 7, 64, 16, False, 16, 16),
        ([4097] + [300] * 7, 64, 16, False, 0, 16),
        ([8193] + [300] * 7, 64, 16, False, 0, 0),  # past 16 waves x 512 tokens: KV splits
        # More than one round of row workgroups: 12 requests of short contexts stay rows, longer
        # ones and more than 512 workgroups (24 requests) take KV splits, beside prefill tiles too.
        ([1000] * 12, 64, 16, False, 16, 16),
        ([2000] * 12, 64, 16, False, 0, 0),
        ([1000] * 24, 64, 16, False, 0, 0),
        ([4096, 1, 300], 64, 16, True, 0, 0),  # asked for KV splits
        ([2000], 256, 16, False, 0, 0),  # head_dim past the workgroup kernel's 128
        ([2000], 128, 8, False, 8, 8),
        ([2000], 64, 32, False, 8, 8),
    ],
)
def test_plan_row_mode_selection(ctx, d, bs, split_rows, row_waves, row_waves_tiles) -> None:
    """Decode rows become workgroups whose waves split the keys and merge in LDS when the fast
    decode kernel takes the shape: one of 16 waves per (request, kv head) when they cover the
    256 CUs in one round (or in two, on contexts of at most 1,536 tokens) and every decode context
    fits 16 waves of at most 256 tokens (512 when the plan puts prefill tiles on a second stream
    beside them), one of 8 waves per part of a context when they would not cover the CUs."""
    n, h = len(ctx), 32
    plan, ws = kernels.make_plan_host(np.arange(n + 1, dtype=np.int32), np.array(ctx, np.int32),
                                      h, h, d, bs, -(-max(ctx) // bs), torch.float16, split_rows)
    assert int(plan[19]) == row_waves
    items, reqs = decode_plan(plan)
    if row_waves and n * h >= 256:
        assert ws == 0 and int(plan[16]) == 0
        assert items.shape[0] == n * h and all(int(nsplit) == 1 for nsplit in reqs[:, 0])
    if row_waves and n * h < 256:
        check_parts(ctx, h, bs, items, reqs, plan)
    if row_waves and d == 64 and bs == 16:
        check_coverage(list(range(n + 1)), ctx, h, h)
    # With a prefill slice of 600 tokens at offset 3000 in the batch.
    qsl = np.array([0, *range(1, n + 1), n + 600], np.int32)
    plan2, _ = kernels.make_plan_host(qsl, np.array([*ctx, 3600], np.int32), h, h, d, bs,
                                      -(-max(*ctx, 3600) // bs), torch.float16, split_rows,
                                      force_overlap=True)
    assert int(plan2[19]) == row_waves_tiles and int(plan2[20]) == 1
    # Planned for one stream (160 tiles do not fill the CUs), the rows run alone after the tiles.
    plan3, _ = kernels.make_plan_host(qsl, np.array([*ctx, 3600], np.int32), h, h, d, bs,
                                      -(-max(*ctx, 3600) // bs), torch.float16, split_rows)
    assert int(plan3[19]) == row_waves and int(plan3[20]) == 0


def _mixed(slices, decodes):
    """query_start_loc / context_lens of prefill slices (tokens, prefix) followed by decodes."""
    q = [c for c, _ in slices] + [1] * len(decodes)
    ctx = [c + p for c, p in slices] + list(decodes)
    return np.concatenate([[0], np.cumsum(q)]).astype(np.int32), np.array(ctx, np.int32)


@pytest.mark.parametrize("slices,decodes,force,overlap", [
    # config 3: 384 tiles (every CU at one workgroup) beside 24 decodes reading 707 MB
    ([(512, 0), (512, 3584), (512, 6656)], "cfg3", False, 1),
    ([(512, 3000)], [3000] * 7, False, 0),  # a serving chunk: 128 tiles
    ([(512, 3000)], [3000] * 7, True, 1),
    ([(512, 0), (512, 3584), (512, 6656)], [100] * 24, False, 0),  # light rows (20 MB)
    ([], [3000] * 7, True, 0),  # no tiles
    ([(512, 3000)], [], True, 0),  # no rows
])
def test_plan_overlap_choice(slices, decodes, force, overlap) -> None:
    """Plan word 20 records whether the batch is planned for tiles beside rows on two streams:
    only when the tiles fill every CU and the rows read at least 256 MiB (or when asked), and
    never without both. The tile split follows the run: toward the 256 slots of one workgroup
    per CU beside the rows, 512 for the one-stream run; no tile item spans more keys than its
    share of the tile work (at least 1,024), and a request's splits are equal 64-key multiples."""
    if decodes == "cfg3":
        decodes = torch.randint(512, 7473, (24,), generator=torch.Generator().manual_seed(3))
        decodes = [int(x) for x in decodes]
    qsl, ctx = _mixed(slices, decodes)
    plan, _ = kernels.make_plan_host(qsl, ctx, 32, 32, 64, 16, -(-int(ctx.max()) // 16),
                                     torch.float16, force_overlap=force)
    assert int(plan[20]) == overlap
    n_tiles = int(plan[2]) - int(plan[13])
    if not slices:
        assert n_tiles == 0
        return
    target = 256 if overlap else 512
    work = sum(-(-c // 128) * 32 * (c + p) for c, p in slices)
    part = -(-max(1024, -(-work // target)) // 64) * 64
    items, reqs = decode_plan(plan)
    expected = 0
    for r, (c, p) in enumerate(slices):
        L = c + p
        n = -(-L // part)
        slen = -(-(-(-L // n)) // 64) * 64
        assert int(reqs[r][1]) == slen and int(reqs[r][0]) == -(-L // slen)
        for t in range(-(-c // 128)):  # splits past a tile's causal limit are skipped
            expected += 32 * min(-(-L // slen), (p + 128 * t + min(128, c - 128 * t) - 1) // slen + 1)
    assert n_tiles == expected
    assert all(int(ke) - int(kb) <= part for _r, _h, _qb, _qc, kb, ke, *_ in
               items[int(plan[13]):].tolist())
