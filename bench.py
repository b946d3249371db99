"""Benchmark of the ragged decoder step on one MI355X.

``python bench.py [--steps K] [--warmup W]`` prints ONE JSON line. The headline workload is
32 decode requests with contexts drawn from U[256, 7472], 32/32 heads of 64,
fp16, a 16,384-block pool (1 GiB per K or V pool) with seeded-shuffled block tables. One step is
the decoder-step hot path on that batch: slot-mapped append of the 32 new K/V tokens, then fused
ragged paged attention over every context. ``value`` is the step's algorithmic KV bytes
(context reads + appended K/V + q/out + block tables) divided by the step time, in GB/s.

Extra fields (same line, tables as ``cols`` + ``rows`` arrays so the whole line stays a few KB):
``cfg3`` (3 prefill slices of 512 + 24 decodes, one step), ``single_seq`` (the reference's
published fused-attention shape: batch 1 and 2 decodes at L in {128 ... 7992}), ``cfg4`` (INT8 /
INT4 quant linears over M in {1, 8, 32, 64, 512, 544}, weight replicas rotated through >= 1 GiB so
the timings are HBM, not Infinity Cache), ``lm_head`` (the fused output head + greedy argmax)
and ``cfg5`` (the 24-layer decoder serving the synthetic Poisson trace).

Timing: W untimed warmup steps, then K steps bracketed by ``torch.cuda.synchronize()`` and HIP
events on the stream the kernels are launched on (torch's current stream). The step's metadata
(block tables, slot mapping, attention plan) is built and uploaded before the timed region, like
every other input; its host cost is reported separately as ``plan_us``.

``cpu_baseline`` (on the line, and inside ``cfg3``, ``cfg4`` and ``cfg5``) times this repository's
CPU restatement of the reference path (the oracle, fp32, the host's cores): the full config-2 and
config-3 steps (gather + SDPA, ``edgerag/cache/paged.py:208-238`` +
``edgerag/core/layers.py:137-167``), every config-4 shape and M (dequantise + ``F.linear``,
``edgerag/core/linear.py:186-196``), and a truncated config-5 decode (one request through the
24-layer decoder oracle), each labelled with what it ran.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from edgerag_amd import kernels  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16
BS = 16
H = 32
D = 64
KV_BYTES_PER_TOKEN = 2 * H * D * 2  # K and V, one layer, fp16 = 8192


# --- workloads -----------------------------------------------------------------------------------


def make_batch(lens, q_lens, num_blocks, seed, device):
    """Pools, disjoint shuffled tables, packed q/new K/V, slot mapping and the attention plan."""
    g = torch.Generator().manual_seed(seed)
    nbs = [math.ceil(L / BS) for L in lens]
    perm = torch.randperm(num_blocks, generator=g).numpy().astype(np.int32)
    bt = np.full((len(lens), max(nbs)), -1, np.int32)
    at = 0
    slots = []
    for r, (L, c, nb) in enumerate(zip(lens, q_lens, nbs)):
        bt[r, :nb] = perm[at : at + nb]
        at += nb
        pos = np.arange(L - c, L)
        slots.append(bt[r, pos // BS].astype(np.int64) * BS + pos % BS)
    slots = np.concatenate(slots).astype(np.int32)
    gd = torch.Generator(device=device).manual_seed(seed)
    shape = (H, num_blocks, BS, D)
    kp = torch.randn(shape, generator=gd, device=device, dtype=torch.float16)
    vp = torch.randn(shape, generator=gd, device=device, dtype=torch.float16)
    T = int(sum(q_lens))
    q = torch.randn(T, H, D, generator=gd, device=device, dtype=torch.float16)
    nk = torch.randn(T, H, D, generator=gd, device=device, dtype=torch.float16)
    nv = torch.randn(T, H, D, generator=gd, device=device, dtype=torch.float16)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    ctx = np.asarray(lens, np.int32)
    plan, (slot_dev,) = kernels.plan_attention(qsl, ctx, bt, H, H, D, BS, torch.float16, device,
                                               [slots])
    # The step's host cost, warm (median of repeated calls): the whole plan_attention (planner,
    # packing, the pinned upload enqueued) and the native planner alone.
    full, planner = [], []
    for _ in range(30):
        t0 = time.perf_counter()
        kernels.plan_attention(qsl, ctx, bt, H, H, D, BS, torch.float16, device, [slots])
        t1 = time.perf_counter()
        kernels.make_plan_host(qsl, ctx, H, H, D, BS, bt.shape[1], torch.float16)
        t2 = time.perf_counter()
        full.append(t1 - t0)
        planner.append(t2 - t1)
    torch.cuda.synchronize()
    out = torch.empty_like(q)
    return dict(kp=kp, vp=vp, q=q, nk=nk, nv=nv, plan=plan, slots=slot_dev, out=out, bt=bt,
                qsl=qsl, lens=lens, q_lens=q_lens, plan_us=float(np.median(full)) * 1e6,
                planner_us=float(np.median(planner)) * 1e6)


def step_bytes(lens, q_lens, bt):
    kv_read = sum(lens) * KV_BYTES_PER_TOKEN
    append = sum(q_lens) * KV_BYTES_PER_TOKEN
    q_out = 2 * sum(q_lens) * H * D * 2
    tables = sum(math.ceil(L / BS) for L in lens) * 4
    return kv_read, append, q_out, tables


def run_step(b):
    """The KV append and the attention of one step, through paged_attention_append: one launch
    for a decode-only batch (the append fused into the decode rows); with prefill tiles, the tiles
    after the append of the new rows on the current stream and the decode rows, appending their
    own positions, on a second one."""
    kernels.paged_attention_append(b["nk"], b["nv"], b["slots"], b["q"], b["kp"], b["vp"],
                                   b["plan"], D**-0.5, out=b["out"])


def time_step(b, steps, warmup):
    """Returns (ms per step, ms per attention launch) from events on the current stream."""
    for _ in range(warmup):
        run_step(b)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    for e0, e1, e2 in ev:
        e0.record()
        e1.record()  # the attention launch carries the append
        run_step(b)
        e2.record()
    torch.cuda.synchronize()
    step_ms = sum(e0.elapsed_time(e2) for e0, _, e2 in ev) / steps
    attn_ms = sum(e1.elapsed_time(e2) for _, e1, e2 in ev) / steps
    wall0 = torch.cuda.Event(enable_timing=True)
    wall1 = torch.cuda.Event(enable_timing=True)
    wall0.record()
    for _ in range(steps):
        run_step(b)
    wall1.record()
    torch.cuda.synchronize()
    return wall0.elapsed_time(wall1) / steps, attn_ms, step_ms


def copy_bandwidth(device, nbytes=1 << 30, iters=20):
    """Read+write GB/s of torch's device copy over 1 GiB: the practical streaming ceiling."""
    src = torch.empty(nbytes // 2, dtype=torch.float16, device=device).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / iters
    return round(2 * nbytes / us / 1e3, 1)


def measured_traffic(name: str) -> int | None:
    """HBM bytes per launch recorded by the rocprofv3 PMC runs summarised in ``profiles/``."""
    path = ROOT / "profiles" / name
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1])
    return None


def cfg2_lens():
    g = torch.Generator().manual_seed(2)
    return torch.randint(256, 7473, (32,), generator=g).tolist()


def cfg3_lens():
    g = torch.Generator().manual_seed(3)
    dec = torch.randint(512, 7473, (24,), generator=g).tolist()
    lens = [512, 3584 + 512, 6656 + 512] + dec
    q_lens = [512, 512, 512] + [1] * 24
    return lens, q_lens


# --- config 4: quant linears ---------------------------------------------------------------------


# --- access-pattern ceilings (edgerag_amd/csrc/probe/edgerag_probe.h) ----------------------------

_PROBE = None


def _probe_call(name: str, *args) -> None:
    """Call an entry point of the bench-only probe library (built beside the product one)."""
    global _PROBE
    import ctypes

    from edgerag_amd._build import PROBE_LIB_PATH

    if _PROBE is None:
        lib = ctypes.CDLL(str(PROBE_LIB_PATH))
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        lib.edgerag_probe_read.argtypes = [vp, i64, i32, i32, vp, vp]
        lib.edgerag_probe_gather.argtypes = [vp, vp, i32, i32, i32, i32, vp, vp]
        lib.edgerag_last_error.restype = ctypes.c_char_p
        _PROBE = lib
    rc = getattr(_PROBE, name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed ({rc}): {_PROBE.edgerag_last_error().decode()}")



def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def probe_read_us(buffers, nbytes, n_launch=256, shapes=((512, 2), (1024, 2), (2048, 1))):
    """Launch-to-launch time of the streaming-read probe over `nbytes` of each buffer in turn
    (graph replay of `n_launch` launches, like the cfg4 timings): the best a kernel that only
    reads the same bytes can do. The fastest of the (workgroups, unroll) launch shapes is kept."""
    from edgerag_amd import _lib

    sink = torch.zeros(1, dtype=torch.int32, device=buffers[0].device)
    best = None
    for wgs, unroll in shapes:
        def launch(buf):
            _probe_call("edgerag_probe_read", buf.data_ptr(), nbytes, wgs, unroll, sink.data_ptr(),
                      _stream())

        launch(buffers[0])
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(n_launch):
                launch(buffers[i % len(buffers)])
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(3):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (3 * n_launch)
        del graph
        best = us if best is None else min(best, us)
    return best


def measure_ceilings(device, gather_bytes):
    """HBM ceilings of the two access patterns on this GPU (rooflines read against them as well as
    against the datasheet 8 TB/s): a 1 GiB contiguous stream, and `gather_bytes` read as random
    2 KiB chunks of a 2 GiB buffer (the paged pool's (head, block) rows) -- the cfg2 decode
    launch's pattern and byte count -- with plain loads and with non-temporal ones (the load
    policy of the decode rows)."""
    from edgerag_amd import _lib

    out = {}
    buf = torch.empty(1 << 30, dtype=torch.uint8, device=device)
    buf.fill_(1)
    big = ((1024, 2), (4096, 2), (8192, 4), (16384, 2))
    out["stream_read_1GiB_gbs"] = round(
        (1 << 30) / probe_read_us([buf], 1 << 30, 8, shapes=big) / 1e3, 1)
    del buf
    pool = torch.empty(2 << 30, dtype=torch.uint8, device=device)
    pool.fill_(1)
    per_wave = 128
    n_chunks = int(gather_bytes // 2048) // per_wave * per_wave
    gen = torch.Generator(device=device).manual_seed(5)
    ids = torch.randint(0, (2 << 30) // 2048, (n_chunks,), generator=gen, device=device,
                        dtype=torch.int32)
    sink = torch.zeros(1, dtype=torch.int32, device=device)

    def gather_gbs(nontemporal):
        def launch():
            _probe_call("edgerag_probe_gather", pool.data_ptr(), ids.data_ptr(),
                        n_chunks // per_wave, per_wave, 2048, nontemporal, sink.data_ptr(),
                        _stream())

        launch()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            launch()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / 10
        return round(n_chunks * 2048 / us / 1e3, 1)

    out["gather_2KiB_gbs"] = gather_gbs(0)
    # Non-temporal loads, as the decode rows read the pools: the ceiling of their pattern.
    out["gather_2KiB_nt_gbs"] = gather_gbs(1)
    del pool, ids
    torch.cuda.empty_cache()
    return out


def vendor_gemm_us(x, packed, scales, k, bits, g, n_w=8, n_launch=64):
    """torch's fp16 ``x @ W^T`` (hipBLASLt) over ``n_w`` dequantised weight replicas, replayed
    from a HIP graph of ``n_launch`` back-to-back launches: average launch-to-launch time, µs.
    The weights are stored (K, N) contiguous, so the product is a plain mm."""
    n_w = min(n_w, packed.shape[0])
    wt = [kernels.dequantize(packed[r], scales[r], k, bits, g).t().contiguous() for r in range(n_w)]
    y = torch.empty(x.shape[0], wt[0].shape[1], device=x.device, dtype=torch.float16)
    for r in range(n_w):
        torch.mm(x, wt[r], out=y)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(n_launch):
            torch.mm(x, wt[i % n_w], out=y)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (3 * n_launch)
    del graph, wt, y
    return us


CFG4_SHAPES = [(2048, 2048, 8, 2048), (2048, 8192, 8, 2048), (8192, 2048, 8, 8192),
               (1152, 1152, 4, 128), (1152, 4608, 4, 128)]
CFG4_MS = (1, 8, 32, 64, 512, 544)


def run_cfg4(device, args):
    """Config 4 as compact rows: [K, N, bits, M, us, frac, ref_us, cpu_us]. ``frac`` is of the
    row's roofline (HBM 8 TB/s for M <= 64, dense fp16 MFMA 2.5 PFLOP/s above); ``ref_us`` is the
    streaming-read probe over the same weight bytes for the HBM rows and torch's fp16 GEMM
    (hipBLASLt) on the dequantised weights for the MFMA rows; ``cpu_us`` the CPU baseline."""
    rows = bench_quant(device)
    cpu = {}
    if not args.no_cpu:
        for r in cpu_quant_rows(CFG4_SHAPES, CFG4_MS):
            cpu[(r["k"], r["n"], r["m"])] = r["us"]
    out = []
    for r in rows:
        ref = r["read_us"] if r["bound"] == "hbm" else r["vendor_fp16_us"]
        out.append([r["k"], r["n"], r["bits"], r["m"], r["us"], r["frac"], ref,
                    cpu.get((r["k"], r["n"], r["m"]))])
    res = {"cols": ["k", "n", "bits", "m", "us", "frac", "ref_us", "cpu_us"], "rows": out}
    if cpu:
        res["cpu_baseline"] = {"unit": "us per call", "cores": cpu_threads(), "kind": "port",
                               "sample": "oracle dequantise + F.linear, fp32, median of >= 20"}
    return res


def bench_quant(device, iters=None):
    """Config 4. Each timing replays a HIP graph of back-to-back launches, one per weight replica
    (>= 1 GiB of distinct packed weights in rotation, so the weights stream from HBM rather than
    the Infinity Cache); the graph removes the host's per-call cost from the launch-to-launch gap.
    ``us`` is the average launch-to-launch time on the GPU, events on the capture stream.
    ``read_us`` is the streaming-read probe over the same packed-weight replicas, the same way:
    the time any kernel needs just to read those bytes at this size (``read_frac`` = read_us /
    us for the HBM-bound rows). For the MFMA-bound rows, ``vendor_fp16_us`` is torch's fp16
    GEMM (hipBLASLt) on the dequantised weights of the same shape, timed the same way:
    what the vendor library needs for the matrix product alone, with no dequantisation."""
    results = []
    for k, n, bits, g in CFG4_SHAPES:
        width = k // 2 if bits == 4 else k
        wbytes = n * width + n * (k // g) * 2
        reps = max(2, math.ceil((1 << 30) / wbytes))
        gen = torch.Generator(device=device).manual_seed(k + n)
        packed = torch.randint(0, 256, (reps, n, width), generator=gen, device=device,
                               dtype=torch.uint8)
        scales = (torch.rand((reps, n, k // g), generator=gen, device=device) * 1e-3 + 1e-4).half()
        read_us = probe_read_us([packed[r] for r in range(reps)], n * width, min(reps, 512))
        for m in CFG4_MS:
            x = torch.randn(m, k, generator=gen, device=device, dtype=torch.float16)
            y = torch.empty(m, n, device=device, dtype=torch.float16)
            n_launch = iters or min(reps, 512)
            for i in range(3):
                kernels.quant_linear(x, packed[i], scales[i], None, k, n, bits, g, out=y)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for i in range(n_launch):
                    r = i % reps
                    kernels.quant_linear(x, packed[r], scales[r], None, k, n, bits, g, out=y)
            graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            n_rep = 3
            e0.record()
            for _ in range(n_rep):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (n_rep * n_launch)
            del graph
            nbytes = wbytes + 2 * m * k + 2 * m * n
            flops = 2 * m * n * k
            gbs = nbytes / us / 1e3
            tflops = flops / us / 1e6
            bound = "hbm" if m <= 64 else "mfma"
            frac = gbs / HBM_PEAK_GBS if bound == "hbm" else tflops / MFMA_F16_PEAK_TFLOPS
            row = dict(k=k, n=n, bits=bits, group=g, m=m, us=round(us, 2),
                       gbs=round(gbs, 1), tflops=round(tflops, 2), bound=bound,
                       frac=round(frac, 4), read_us=round(read_us, 2))
            if bound == "hbm":
                row["read_frac"] = round(read_us / us, 4)
            else:
                row["vendor_fp16_us"] = round(vendor_gemm_us(x, packed, scales, k, bits, g), 2)
            results.append(row)
        del packed, scales
        torch.cuda.empty_cache()
    return results


def bench_lm_head(device, vocab=49152, k=2048, ms=(1, 8, 16), reps=3):
    """The output head of a decode step (config 5's lm_head: fp16 49152 x 2048, 201 MB): the
    fused GEMV + greedy argmax (edgerag_lm_head_argmax) against torch's fp16 F.linear (hipBLASLt)
    followed by edgerag_argmax_rows, both replayed from HIP graphs over ``reps`` weight replicas
    (more bytes than the Infinity Cache holds); ``read_us`` is the streaming-read probe over the
    same replicas."""
    gen = torch.Generator(device=device).manual_seed(11)
    ws = [(torch.randn(vocab, k, generator=gen, device=device) * 0.02).half() for _ in range(reps)]
    wbytes = vocab * k * 2
    read_us = probe_read_us(ws, wbytes, 4 * reps, shapes=((1024, 2), (2048, 1), (4096, 1)))
    rows = []
    for m in ms:
        x = torch.randn(m, k, generator=gen, device=device).half()
        logits = torch.empty(m, vocab, dtype=torch.float16, device=device)
        tokens = torch.empty(m, dtype=torch.int32, device=device)

        def fused(i):
            kernels.lm_head_argmax(x, ws[i % reps], logits, tokens)

        def vendor(i):
            torch.mm(x, ws[i % reps].t(), out=logits)  # what F.linear(x, W) runs
            kernels.argmax_rows(logits, out=tokens)

        res = {}
        for name, fn in (("fused", fused), ("vendor", vendor)):
            for i in range(reps):
                fn(i)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            n_launch = 24
            with torch.cuda.graph(graph):
                for i in range(n_launch):
                    fn(i)
            graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(5):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
            res[name] = e0.elapsed_time(e1) * 1e3 / (5 * n_launch)
            del graph
        nbytes = wbytes + 2 * m * k + 2 * m * vocab
        rows.append([m, round(res["fused"], 2), round(res["vendor"], 2), round(read_us, 2),
                     round(nbytes / res["fused"] / 1e3 / HBM_PEAK_GBS, 4)])
    del ws
    torch.cuda.empty_cache()
    return {"cols": ["m", "us", "vendor_us", "read_us", "frac"], "rows": rows}


# --- CPU baselines ---------------------------------------------------------------------------------
#
# This repository's CPU restatement of the reference path (the oracle, PyTorch on the host's cores,
# fp32 as the reference's own CPU tests run): gather + SDPA for attention
# (edgerag/cache/paged.py:208-238, edgerag/core/layers.py:137-167), dequantise + F.linear for the
# quant linears (edgerag/core/linear.py:186-196), the decoder forward one request at a time for
# config 5 (edgerag/core/model.py:72-152, edgerag/serve/executor.py:113-156). Timing follows the
# reference's rules (bench/metrics.py:1-12): warmup discarded, median of >= 20 runs.


def cpu_threads() -> int:
    cores = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        cores = min(cores, int(env))
    torch.set_num_threads(cores)
    return cores


def _median_runs(fn, min_runs=20, budget_s=3.0):
    fn()  # warmup, discarded
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= 200:
            break
    return float(np.median(times)), len(times)


def cpu_attention_step(lens, q_lens, seed):
    """One ragged step on the CPU oracle: slot writes of the new K/V, then per request gather +
    causal SDPA (fp32). Returns (median s, runs, algorithmic bytes as on the GPU)."""
    from oracle import attention as oa
    from oracle import paged as op

    nbs = [math.ceil(L / BS) for L in lens]
    g = torch.Generator().manual_seed(seed)
    kp = torch.randn(H, sum(nbs), BS, D, generator=g)
    vp = torch.randn(H, sum(nbs), BS, D, generator=g)
    tables, at = [], 0
    for nb in nbs:
        tables.append(list(range(at, at + nb)))
        at += nb
    qsl = [0]
    for c in q_lens:
        qsl.append(qsl[-1] + c)
    q = torch.randn(qsl[-1], H, D, generator=g)
    new = torch.randn(qsl[-1], H, D, generator=g)

    def once():
        for r, (L, c, t) in enumerate(zip(lens, q_lens, tables)):
            src = new[qsl[r] : qsl[r + 1]].transpose(0, 1)[None]  # (1, H, c, D)
            op.write_slots(kp, src, t, L - c)
            op.write_slots(vp, src, t, L - c)
        oa.ragged_reference(q, kp, vp, qsl, lens, tables, D**-0.5)

    med, runs = _median_runs(once)
    kv, ap, qo, tb = step_bytes(lens, q_lens, np.zeros((len(lens), max(nbs)), np.int32))
    return med, runs, kv + ap + qo + tb


def cpu_quant_rows(shapes, ms):
    """Dequantise + F.linear (fp32 activations, the oracle's quant_linear_reference) per cfg4
    shape and M; microseconds per call."""
    from oracle import quant as oq

    rows = []
    for k, n, bits, grp in shapes:
        cfg = oq.QuantConfig(grp, bits)
        g = torch.Generator().manual_seed(k + n)
        packed, scales = oq.quantize_for_layer(torch.randn(n, k, generator=g) * 0.02, cfg)
        for m in ms:
            x = torch.randn(m, k, generator=g)
            med, runs = _median_runs(
                lambda: oq.quant_linear_reference(x, packed, scales, None, k, cfg), budget_s=0.3)
            rows.append(dict(k=k, n=n, bits=bits, group=grp, m=m, us=round(med * 1e6, 1),
                             runs=runs))
    return rows


def cpu_decoder_tok_s(model, prompt_len=512, new_tokens=16, seed=5):
    """Config 5, truncated: one request of ``prompt_len`` random ids, greedy ``new_tokens``
    through the 24-layer decoder oracle (the same quantised weights, dequantised to fp32), one
    request per forward as the reference executor runs it. Output tokens / wall time."""
    from oracle import model as om

    oracle = om.OracleDecoder(model, torch.float32)  # dequantised once, not timed
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(1, model.spec.vocab_size - 1, (prompt_len,), generator=g).tolist()

    def once(n_prompt, n_new):
        t0 = time.perf_counter()
        oracle.reset()
        out = [int(oracle.forward(prompt[:n_prompt])[-1].argmax())]
        t1 = time.perf_counter()
        while len(out) < n_new:
            out.append(int(oracle.forward([out[-1]])[-1].argmax()))
        t2 = time.perf_counter()
        return t2 - t0, t2 - t1

    once(64, 2)  # warmup, discarded (bench/metrics.py:1-12)
    runs = [once(prompt_len, new_tokens) for _ in range(3)]
    total = float(np.median([r[0] for r in runs]))
    dec = float(np.median([r[1] for r in runs]))
    del oracle
    return {"value": round(new_tokens / total, 3), "unit": "output tok/s",
            "decode_tok_s": round((new_tokens - 1) / dec, 3), "runs": 3,
            "sample": f"1 request, {prompt_len}-token prompt, {new_tokens} tokens, 24-layer "
            "fp32 oracle, median of 3 after a warmup"}


def run_cfg3(device, args):
    """Config 3: 3 prefill slices + 24 decodes in one step (append + attention)."""
    lens3, q3 = cfg3_lens()
    b3 = make_batch(lens3, q3, 16384, 3, device)
    s3, a3, _ = time_step(b3, max(5, args.steps // 2), max(2, args.warmup // 2))
    kv3, ap3, qo3, tb3 = step_bytes(lens3, q3, b3["bt"])
    step_bytes_total = kv3 + ap3 + qo3 + tb3
    res = {
        "ms_per_step": round(s3, 4),
        "step_bytes": int(step_bytes_total),
        "gbs": round(step_bytes_total / (s3 * 1e-3) / 1e9, 1),
        "hbm_frac": round(step_bytes_total / (s3 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "attn_us": round(a3 * 1e3, 1),  # the append + attention launches (one call)
        "items": b3["plan"].n_items,
    }
    del b3
    torch.cuda.empty_cache()
    if not args.no_cpu:
        med, runs, nbytes = cpu_attention_step(lens3, q3, 8)
        res["cpu_baseline"] = {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s",
                               "cores": cpu_threads(), "kind": "port", "runs": runs}
    return res


# --- single-sequence fused decode attention (the reference's published shape) --------------------

SINGLE_SEQ_LENS = (128, 512, 1024, 2048, 4096, 6758, 7992)


def bench_single_seq(device, lens=SINGLE_SEQ_LENS, batch=1, num_blocks=16384):
    """``fused_paged_attention`` at the reference's published shape (``CONTEXT.md:1584-1592``):
    one (or ``batch``) decode query, 32/32 heads of 64, fp16, 16-token blocks, at each context
    length. Every launch of a replayed HIP graph attends a different sequence (disjoint shuffled
    block tables over a 16,384-block pool, 2 GiB of K + V), so the K/V stream from HBM, not the
    Infinity Cache. ``us`` is the launch-to-launch time (the merge launch included where the plan
    cuts contexts into parts); bytes = K/V read + q/out + block table."""
    gd = torch.Generator(device=device).manual_seed(17)
    shape = (H, num_blocks, BS, D)
    kp = torch.randn(shape, generator=gd, device=device, dtype=torch.float16)
    vp = torch.randn(shape, generator=gd, device=device, dtype=torch.float16)
    g = torch.Generator().manual_seed(17)
    rows = []
    for L in lens:
        nb = math.ceil(L / BS)
        # >= 1.2 GB of distinct K/V per replay, or the whole pool.
        n_seq = min(num_blocks // (nb * batch),
                    max(64, math.ceil(1.2e9 / (batch * L * KV_BYTES_PER_TOKEN))))
        n_launch = max(64, n_seq)
        perm = torch.randperm(num_blocks, generator=g).numpy().astype(np.int32)
        plans, qs, outs = [], [], []
        for i in range(n_seq):
            bt = perm[i * nb * batch : (i + 1) * nb * batch].reshape(batch, nb)
            qsl = np.arange(batch + 1, dtype=np.int32)
            plan, _ = kernels.plan_attention(qsl, np.full(batch, L, np.int32), bt, H, H, D, BS,
                                             torch.float16, device)
            plans.append(plan)
            qs.append(torch.randn(batch, H, D, generator=gd, device=device, dtype=torch.float16))
            outs.append(torch.empty(batch, H, D, device=device, dtype=torch.float16))
        for i in range(n_seq):
            kernels.paged_attention(qs[i], kp, vp, plans[i], D**-0.5, out=outs[i])
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(n_launch):
                j = i % n_seq
                kernels.paged_attention(qs[j], kp, vp, plans[j], D**-0.5, out=outs[j])
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (5 * n_launch)
        del graph
        nbytes = batch * (L * KV_BYTES_PER_TOKEN + 2 * H * D * 2 + nb * 4)
        ph = plans[0].plan_host
        rows.append([L, round(us, 2), round(nbytes / us / 1e3, 1),
                     round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), int(ph[2]), int(ph[16] > 0)])
    del kp, vp
    torch.cuda.empty_cache()
    return rows


SINGLE_SEQ_COLS = ["L", "us", "gbs", "frac", "items", "merge"]


def run_single_seq(device):
    return {"cols": SINGLE_SEQ_COLS, "b1": bench_single_seq(device),
            "b2": bench_single_seq(device, batch=2)}


# --- config 5: end-to-end serving ---------------------------------------------------------------


def run_cfg5(device, n_requests: int = 64, cpu: bool = True):
    """Config 5: the 24-layer SmolLM2-1.7B-shaped decoder (INT8 per-channel linears, fp16
    embeddings / norms / lm_head, random init) serving a seeded Poisson trace (12 req/min,
    lognormal prompts median 3000 clamped to [256, 7472], 64-256 greedy tokens) through the
    scheduler (max batch 8, one 512-token prefill chunk per iteration, CoW reserve 4) and the
    ragged executor. ``offered_load`` replays the arrivals on a virtual clock (idle gaps skipped);
    ``saturated`` submits every request at t = 0 (capacity)."""
    from edgerag_amd.cache.allocator import BlockAllocator
    from edgerag_amd.core.model import EdgeRagDecoder
    from edgerag_amd.core.spec import SMOLLM2_1_7B
    from edgerag_amd.sched.scheduler import Scheduler, SchedulerConfig
    from edgerag_amd.serve.executor import ModelExecutor
    from edgerag_amd.serve.replay import poisson_arrivals, replay, synthetic_requests

    spec = SMOLLM2_1_7B
    model = EdgeRagDecoder(spec, bits=8, group_size=None, device=device, dtype=torch.float16)
    model.init_random(seed=5)
    torch.cuda.synchronize()
    num_blocks = 8 * math.ceil((7472 + 256) / BS) + 64
    alloc = BlockAllocator(num_blocks, BS)
    executor = ModelExecutor(model, spec, alloc, device, torch.float16, chunk_size=512)
    warm = synthetic_requests(2, spec.vocab_size, seed=99, median=700, sigma=0.01, min_new=4,
                              max_new=4)
    replay(Scheduler(alloc, SchedulerConfig()), executor, warm, None, "saturated")
    reqs = synthetic_requests(n_requests, spec.vocab_size, seed=5)
    arrivals = poisson_arrivals(len(reqs), 12.0 / 60.0, seed=5)
    offered = replay(Scheduler(alloc, SchedulerConfig()), executor, reqs, arrivals, "virtual")
    reqs = synthetic_requests(n_requests, spec.vocab_size, seed=5)
    saturated = replay(Scheduler(alloc, SchedulerConfig()), executor, reqs, None, "saturated")
    def brief(summary):
        keep = ("output_tok_per_s", "iterations", "iteration_ms_p50", "iteration_ms_p99",
                "ttft_s_p50", "ttft_s_p99", "gpu_busy_s")
        return {k: summary[k] for k in keep}

    res = {"requests": n_requests, "offered_load": brief(offered.summary()),
           "saturated": brief(saturated.summary()), "weight_bytes": model.weight_bytes()}
    if cpu:
        del executor
        torch.cuda.empty_cache()
        res["cpu_baseline"] = dict(cpu_decoder_tok_s(model), cores=cpu_threads(), kind="port")
    return res


def run_decode_b1(device, prompt: int = 3000, steps: int = 300):
    """The config-5 decoder decoding one request: a ``prompt``-token prompt prefilled in 512-token
    chunks, then ``steps`` greedy decode iterations replayed from graphs (the offered-load case:
    almost every iteration of the config-5 trace has one running request). Reports the
    iteration time as ``replay`` measures it (execute + sync)."""
    from edgerag_amd.cache.allocator import BlockAllocator
    from edgerag_amd.core.model import EdgeRagDecoder
    from edgerag_amd.core.spec import SMOLLM2_1_7B
    from edgerag_amd.sched.request import Request
    from edgerag_amd.sched.scheduler import Scheduler, SchedulerConfig
    from edgerag_amd.serve.executor import ModelExecutor, apply_output

    spec = SMOLLM2_1_7B
    model = EdgeRagDecoder(spec, bits=8, group_size=None, device=device, dtype=torch.float16)
    model.init_random(seed=5)
    alloc = BlockAllocator(math.ceil((prompt + steps) / BS) + 64, BS)
    executor = ModelExecutor(model, spec, alloc, device, torch.float16, chunk_size=512)
    sched = Scheduler(alloc, SchedulerConfig(max_batch_size=1))
    g = torch.Generator().manual_seed(1)
    sched.add_request(Request("r0", torch.randint(1, spec.vocab_size - 1, (prompt,),
                                                  generator=g).tolist(), max_new_tokens=steps))
    times = []
    while sched.has_work:
        batch = sched.schedule()
        t0 = time.perf_counter()
        out = executor.execute(batch)
        torch.cuda.synchronize()
        if not batch.prefill:
            times.append((time.perf_counter() - t0) * 1e3)
        apply_output(sched, batch, out)
    t = np.array(times[20:])
    return {"prompt": prompt, "steps": len(times), "graph_steps": executor.graph_steps,
            "iteration_ms_p50": round(float(np.median(t)), 3),
            "iteration_ms_p99": round(float(np.percentile(t, 99)), 3)}


# --- main ------------------------------------------------------------------------------------------


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-extra", action="store_true", help="skip configs 3 and 4")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-cfg5", action="store_true", help="skip the end-to-end serving run")
    ap.add_argument("--cfg5-requests", type=int, default=64)
    ap.add_argument("--record", default=None,
                    help="also write the full (uncompacted) record of the run to this JSON file")
    ap.add_argument("--only", choices=["cfg3", "cfg4", "cfg5", "lm_head", "single_seq",
                                       "decode_b1"],
                    default=None,
                    help="run just one secondary config (for profiling); prints its record")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the ragged decoder step has no "
                          "multi-GPU path here (sharding is design-only); run with --gpus 1"}))
        sys.exit(2)
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.only == "cfg3":
        print(json.dumps({"cfg3": run_cfg3(device, args)}), flush=True)
        return
    if args.only == "cfg4":
        print(json.dumps({"cfg4": run_cfg4(device, args)}), flush=True)
        return
    if args.only == "lm_head":
        print(json.dumps({"lm_head": bench_lm_head(device)}), flush=True)
        return
    if args.only == "single_seq":
        print(json.dumps({"single_seq": run_single_seq(device)}), flush=True)
        return
    if args.only == "cfg5":
        print(json.dumps({"cfg5": run_cfg5(device, args.cfg5_requests, not args.no_cpu)}),
              flush=True)
        return
    if args.only == "decode_b1":
        print(json.dumps({"decode_b1": run_decode_b1(device)}), flush=True)
        return

    lens = cfg2_lens()
    b = make_batch(lens, [1] * 32, 16384, 2, device)
    step_ms, attn_ms, step_ev_ms = time_step(b, args.steps, args.warmup)
    kv_read, append, q_out, tables = step_bytes(lens, [1] * 32, b["bt"])
    total = kv_read + append + q_out + tables
    # The decode-only cfg2 step runs the append inside the attention launch: its bytes count there.
    attn_bytes = kv_read + q_out + tables + append
    gbs = total / (step_ms * 1e-3) / 1e9
    attn_gbs = attn_bytes / (attn_ms * 1e-3) / 1e9
    line = {
        "metric": "paged-attn step KV GB/s (% HBM peak); quant GEMV GB/s; decoder output tok/s",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) pools/queries, seeded-shuffled block tables)",
        "config": {
            "workload": "cfg2: KV append + ragged paged attention, 32 decodes, L~U[256,7472], "
            "32/32 heads, d64, bs16, 16384-block pool",
            "context_tokens": int(sum(lens)),
            "step_bytes": int(total),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "plan_us": round(b["plan_us"], 1),
            "planner_us": round(b["planner_us"], 1),
            "attn_items": b["plan"].n_items,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "attn_decode_kernel (append fused) + attn_combine_kernel",
            "achieved": round(attn_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic("attn_decode_cfg2.md"),
            "algorithmic_bytes": int(attn_bytes),
            "launch_us": round(attn_ms * 1e3, 2),
        },
    }
    del b
    torch.cuda.empty_cache()
    line["config"]["copy_gbs_1gib"] = copy_bandwidth(device)
    ceilings = measure_ceilings(device, attn_bytes)
    line["ceilings"] = ceilings
    line["roofline"]["frac_of_gather_ceiling"] = round(attn_gbs / ceilings["gather_2KiB_nt_gbs"], 4)
    torch.cuda.empty_cache()
    if not args.no_cpu:
        med, runs, nbytes = cpu_attention_step(lens, [1] * 32, 7)
        line["cpu_baseline"] = {
            "value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": cpu_threads(),
            "kind": "port", "ms_per_step": round(med * 1e3, 2),
            "sample": f"the full cfg2 step (32 requests): slot writes + gather + SDPA per "
            f"request, fp32 oracle, median of {runs} runs",
        }
    if not args.no_extra:
        line["cfg3"] = run_cfg3(device, args)
        line["single_seq"] = run_single_seq(device)
        line["cfg4"] = run_cfg4(device, args)
        line["lm_head"] = bench_lm_head(device)
        if not args.no_cfg5:
            line["cfg5"] = run_cfg5(device, args.cfg5_requests, not args.no_cpu)
    if args.record:
        with open(args.record, "w") as f:
            json.dump(line, f, indent=1)
    print(json.dumps(compact_line(line), separators=(",", ":")), flush=True)


def _sig3(v: float) -> float:
    """v to 3 significant digits (timings in the compact record)."""
    return float(f"{v:.3g}")


def compact_line(line: dict) -> dict:
    """The record printed by a full run, small enough (about 1.8 KB) that the last 2,000
    characters of the run's output hold all of it: the contract fields, the cfg2 roofline and CPU
    baseline, and every secondary table as column lists (``--only <config>`` prints a config's
    full record)."""
    out = {k: line[k] for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup",
                                "ms_per_step", "higher_is_better", "scaling", "vs_baseline",
                                "dtype")}
    out["data"] = "synthetic (seeded N(0,1), shuffled block tables)"
    c = line["config"]
    out["config"] = {"workload": "cfg2: append+paged attn, 32 decodes L~U[256,7472], 32/32h d64 "
                     "bs16", "context_tokens": c["context_tokens"],
                     "step_bytes": c["step_bytes"], "hbm_frac": c["hbm_frac"]}
    r = line["roofline"]
    out["roofline"] = {k: r[k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic")}
    out["roofline"]["launch_us"] = r["launch_us"]
    if "frac_of_gather_ceiling" in r:
        out["roofline"]["gather_frac"] = r["frac_of_gather_ceiling"]
    if "cpu_baseline" in line:
        cb = line["cpu_baseline"]
        out["cpu_baseline"] = {"value": cb["value"], "unit": cb["unit"], "cores": cb["cores"],
                               "kind": cb["kind"], "sample": "cfg2 step, fp32 oracle, median"}
    if "cfg3" in line:
        c3 = line["cfg3"]
        out["cfg3"] = {"ms_per_step": c3["ms_per_step"], "hbm_frac": c3["hbm_frac"]}
        if "cpu_baseline" in c3:
            out["cfg3"]["cpu_gbs"] = c3["cpu_baseline"]["value"]
    if "single_seq" in line:
        b1 = line["single_seq"]["b1"]
        out["single_seq"] = {"L": [row[0] for row in b1], "us": [_sig3(row[1]) for row in b1],
                             "frac": [round(row[3], 3) for row in b1]}
    if "cfg4" in line:
        # Per shape "KxN/bits": us at each M, then the read probe (M <= 64) and hipBLASLt fp16 at
        # each M >= 512 as "ref".
        ms = sorted({row[3] for row in line["cfg4"]["rows"]})
        us, ref, cpu = {}, {}, {}
        for k, n, bits, m, t, _frac, rf, cu in line["cfg4"]["rows"]:
            key = f"{k}x{n}/{bits}"
            us.setdefault(key, []).append(_sig3(t))
            refs = ref.setdefault(key, [])
            if m > 64 or not refs:  # the read probe is the same bytes at every M <= 64
                refs.append(_sig3(rf))
            if m == 1 and cu is not None:
                cpu[key] = round(cu)
        out["cfg4"] = {"m": ms, "us": us, "ref": ref}
        if cpu:
            out["cfg4"]["cpu_us_m1"] = cpu
    if "lm_head" in line:
        rows = line["lm_head"]["rows"]
        out["lm_head"] = {"m": [row[0] for row in rows], "us": [row[1] for row in rows],
                          "vendor_us": [row[2] for row in rows], "read_us": rows[0][3]}
    if "cfg5" in line:
        c5 = line["cfg5"]
        def brief(s):
            return {"tok_s": round(s["output_tok_per_s"], 1), "p50_ms": s["iteration_ms_p50"],
                    "p99_ms": s["iteration_ms_p99"], "ttft_p50_s": s["ttft_s_p50"]}
        out["cfg5"] = {"offered": brief(c5["offered_load"]), "saturated": brief(c5["saturated"])}
        if "cpu_baseline" in c5:
            out["cfg5"]["cpu_tok_s"] = c5["cpu_baseline"]["value"]
    return out


if __name__ == "__main__":
    main()
