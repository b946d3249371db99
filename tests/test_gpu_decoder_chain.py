"""The paths the serving benchmarks time, at their real shapes, against the CPU oracle.

* ``edgerag_paged_attention_fixed`` (the graph-replayed decode attention of every config-5 decode
  iteration) on contexts up to 7,472 tokens: several KV splits per request, the split merge reading
  its row count from the device plan header, one captured graph replayed across plans with
  different split counts.
* The fused decode chain of a decoder layer at the SmolLM2-1.7B width through ``ModelExecutor``
  with graph replay: normed-input q/k/v projection + RoPE + KV append, residual epilogues, SwiGLU
  epilogue, fixed-capacity attention; every step's logits against ``OracleDecoder`` (fp32).
* The 24-layer SmolLM2-1.7B-shaped decoder on two short requests.
* ``paged_attention_append`` (the timed config-2 launch) on the full config-2 workload.
* Attention at block sizes other than 16 (the reference keeps block size a parameter).

Tolerances are written where they are used: attention fp16 atol 2e-3 / rtol 1e-2 (north_star);
decoder logits max |d| <= 2e-2 * max |ref| + 2e-2 (fp16 activations against fp32).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from edgerag_amd import kernels
from edgerag_amd.cache.allocator import BlockAllocator
from edgerag_amd.cache.fused import ragged_paged_attention
from edgerag_amd.core.model import EdgeRagDecoder
from edgerag_amd.core.spec import SMOLLM2_1_7B, ModelSpec
from edgerag_amd.sched.request import Request
from edgerag_amd.sched.scheduler import Scheduler, SchedulerConfig
from edgerag_amd.serve.executor import ModelExecutor, drive
from oracle import attention as oa
from oracle import model as om
from oracle import paged as op
from tests.conftest import seeded

pytestmark = pytest.mark.gpu

FP16_TOL = dict(rtol=1e-2, atol=2e-3)
FP32_TOL = dict(rtol=1e-5, atol=1e-5)


def _tables(lens, bs, num_blocks, g):
    nbs = [math.ceil(L / bs) for L in lens]
    perm = torch.randperm(num_blocks, generator=g).tolist()
    tables, at = [], 0
    for nb in nbs:
        tables.append(perm[at : at + nb])
        at += nb
    bt = np.full((len(lens), max(nbs + [1])), -1, np.int32)
    for r, t in enumerate(tables):
        bt[r, : len(t)] = t
    return tables, bt


# --- fixed-capacity attention (graph replay) at long contexts -----------------------------------


@pytest.mark.parametrize("split_rows", [False, True])
def test_fixed_attention_long_contexts_split_merge_and_graph_replays(device, split_rows) -> None:
    """Every row mode of the fixed launch, switching from step to step as the planner picks
    them: KV splits merged by the combine launch (which reads its row count from the device
    plan header) for long contexts, workgroup-split rows (16 waves per (request, head), merged in
    LDS) when every context is short, and workgroups over parts of the contexts merged by the
    combine launch when the batch is small. One graph per mode replays every plan of that
    mode."""
    n_q = n_kv = 32
    d, bs, cap = 64, 16, 8
    max_blocks = math.ceil(7472 / bs)
    NB = cap * max_blocks + 16
    gd = torch.Generator(device=device).manual_seed(41)
    kp = torch.randn((n_kv, NB, bs, d), generator=gd, device=device, dtype=torch.float16)
    vp = torch.randn((n_kv, NB, bs, d), generator=gd, device=device, dtype=torch.float16)
    fx = kernels.FixedAttention(device, n_q, n_kv, d, bs, torch.float16, cap, max_blocks, [],
                                split_rows=split_rows)
    q_static = torch.zeros((cap, n_q, d), device=device, dtype=torch.float16)
    out = torch.zeros_like(q_static)
    plans = {
        "A": [7472, 6000, 300, 4100, 257, 5000, 7000, 1024],
        "B": [7472, 2000, 100],
        "C": [256, 3000, 7471, 90, 1800],
        "D": [4096, 17, 1000, 2500, 1, 4000, 33, 700],  # every context short
        "E": [300, 16, 3000],
    }
    g = seeded(41)
    cases = {}
    for name, lens in plans.items():
        tables, bt = _tables(lens, bs, NB, g)
        qsl = np.arange(len(lens) + 1, dtype=np.int32)
        q = torch.randn((len(lens), n_q, d), generator=g).half()
        plan_host, _ = kernels.make_plan_host(qsl, np.asarray(lens, np.int32), n_q, n_kv, d, bs,
                                              max_blocks, torch.float16, split_rows)
        cases[name] = (lens, tables, bt, qsl, q, plan_host)
    # A: 8 requests with a context past 16 waves x 256 tokens: KV splits and merge rows. B, C,
    # E: 3-5 requests, fewer workgroups than CUs: workgroups of 8 waves over parts of the
    # contexts, merged by the combine launch. D: 8 short contexts: a workgroup of 16 waves per
    # (request, head), no merge.
    for name in "ABCDE":
        plan = cases[name][5]
        if split_rows or name == "A":
            assert int(plan[19]) == 0 and int(plan[16]) > 0
        elif name == "D":
            assert int(plan[19]) == 16 and int(plan[6]) == 0
        else:
            assert int(plan[19]) == 8 and int(plan[16]) > 0
    # B, C, E share one launch mode; their items, merge rows and partials (read on the device)
    # differ.
    assert len({(int(cases[n][5][6]), int(cases[n][5][13]), int(cases[n][5][16]))
                for n in "BCE"}) == 3

    kp_cpu, vp_cpu = kp.cpu(), vp.cpu()
    graphs = {}
    for name in ["A", "D", "B", "C", "E", "A", "D", "C", "B", "E"]:
        lens, tables, bt, qsl, q, _ = cases[name]
        torch.cuda.synchronize()  # update() reuses its pinned staging buffer
        assert fx.update(qsl, np.asarray(lens, np.int32), bt, [])
        plan = cases[name][5]
        assert fx.mode == (int(plan[19]), int(plan[16]) > 0, int(plan[21]))
        # Parts of few contexts sit in 16 fixed slots per (token, head) (32 kv heads).
        assert int(plan[21]) == (16 if fx.mode[0] == 8 else 0)
        q_static.zero_()
        q_static[: len(lens)].copy_(q.to(device))
        out.fill_(float("nan"))
        if fx.mode not in graphs:
            side = torch.cuda.Stream(device)
            side.wait_stream(torch.cuda.current_stream(device))
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side):
                fx.launch(q_static, kp, vp, 0.125, out)  # eager once before the capture
                with torch.cuda.graph(graph, stream=side):
                    fx.launch(q_static, kp, vp, 0.125, out)
            torch.cuda.current_stream(device).wait_stream(side)
            graphs[fx.mode] = graph
            out.fill_(float("nan"))
        print(f"fixed attention replay, plan {name}: {len(lens)} requests, mode {fx.mode}",
              flush=True)
        graphs[fx.mode].replay()
        torch.cuda.synchronize()
        got = out[: len(lens)].clone()
        eager_plan, _ = kernels.plan_attention(qsl, np.asarray(lens, np.int32), bt, n_q, n_kv, d,
                                               bs, torch.float16, device, split_rows=split_rows)
        eager = kernels.paged_attention(q.to(device), kp, vp, eager_plan, 0.125)
        torch.cuda.synchronize()
        # The same kernels over the same items.
        assert torch.equal(got, eager), f"plan {name}: replay differs from the eager launch"
        expected = oa.ragged_reference(q, kp_cpu, vp_cpu, qsl.tolist(), lens, tables, 0.125)
        torch.testing.assert_close(got.float().cpu(), expected, **FP16_TOL)


def test_fixed_slotted_merge_fails_loudly_on_a_mismatched_plan(device) -> None:
    """The slotted merge launch reads no plan entry: a staged plan whose slot count (word 21)
    differs from the launch's gives NaN rows instead of a merge over the wrong slots."""
    n_q = n_kv = 32
    d, bs, cap = 64, 16, 2
    max_blocks = math.ceil(3000 / bs)
    NB = cap * max_blocks + 16
    gd = torch.Generator(device=device).manual_seed(43)
    kp = torch.randn((n_kv, NB, bs, d), generator=gd, device=device, dtype=torch.float16)
    vp = torch.randn((n_kv, NB, bs, d), generator=gd, device=device, dtype=torch.float16)
    fx = kernels.FixedAttention(device, n_q, n_kv, d, bs, torch.float16, cap, max_blocks, [])
    _, bt = _tables([3000], bs, NB, seeded(43))
    qsl = np.array([0, 1], np.int32)
    assert fx.update(qsl, np.array([3000], np.int32), bt, [])
    assert fx.mode == (8, True, 16)
    q = torch.randn((cap, n_q, d), generator=gd, device=device, dtype=torch.float16)
    out = torch.full_like(q, float("nan"))
    fx.launch(q, kp, vp, 0.125, out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out[:1]).all())
    fx.plan[21] = 0  # the staged plan now claims unslotted partials
    out.fill_(0.0)
    fx.launch(q, kp, vp, 0.125, out)
    torch.cuda.synchronize()
    assert bool(torch.isnan(out[:1]).all())


# --- the decoder's fused decode chain at full width ---------------------------------------------


def _run_recording(model, spec, prompts, max_new, chunk, device, num_blocks, graphs=True):
    """Drive the executor; return per-request [(token, logits row)] in generation order."""
    alloc = BlockAllocator(num_blocks, 16)
    executor = ModelExecutor(model, spec, alloc, device, model.dtype, chunk_size=chunk,
                             decode_graphs=graphs)
    sched = Scheduler(alloc, SchedulerConfig(max_batch_size=8))
    reqs = [Request(f"r{i}", p, max_new_tokens=n) for i, (p, n) in enumerate(zip(prompts, max_new))]
    for r in reqs:
        sched.add_request(r)
    record: dict[str, list[tuple[int, torch.Tensor]]] = {r.request_id: [] for r in reqs}

    def on_step(batch, output):
        if not output.tokens:  # a prefill chunk that emits nothing
            return
        logits = executor.last_logits.float().cpu()
        for row, (rid, token) in enumerate(output.tokens.items()):
            record[rid].append((token, logits[row]))

    drive(sched, executor, on_step=on_step)
    return reqs, record, alloc, executor


def _check_against_oracle(oracle, prompt, steps, tag):
    """Teacher-forced: prefill the prompt (in 512-token chunks, which keeps the oracle's logits
    and masks small), then feed the GPU's own tokens, comparing every step's logits (the GPU's
    greedy choices may differ from the oracle's only at near-ties)."""
    oracle.reset()
    for start in range(0, len(prompt), 512):
        ref = oracle.forward(prompt[start : start + 512])[-1]
    worst = 0.0
    for i, (token, got) in enumerate(steps):
        err = float((got - ref).abs().max())
        bound = 2e-2 * float(ref.abs().max()) + 2e-2
        worst = max(worst, err / bound)
        assert err <= bound, f"{tag} step {i}: max |d| {err:.4g} > {bound:.4g}"
        top2 = torch.topk(ref, 2).values
        if float(top2[0] - top2[1]) > 0.1:
            assert token == int(ref.argmax()), f"{tag} step {i}: greedy token differs"
        ref = oracle.forward([token])[-1]
    print(f"{tag}: worst error / bound = {worst:.3f}", flush=True)


def test_fused_decode_chain_at_smollm2_width_matches_the_oracle(device) -> None:
    """Two layers of the 1.7B shape, INT8 per-channel, fp16, random norm weights: prompts run as
    chunked prefill (512 + 18 tokens, then the others), decode iterations replay from HIP graphs
    through the normed-input / residual / SwiGLU / RoPE-append epilogues and the fixed-capacity
    attention. Every emitted token's logits are checked against the oracle."""
    spec = ModelSpec("smol2", "llama", 2, 2048, 32, 32, 64, 49152, 8192, 130000.0,
                     intermediate_size=8192)
    weights = om.random_weights(spec, 7, 8, None)
    model = EdgeRagDecoder(spec, 8, None, device, torch.float16)
    model.load_quantized(weights)
    assert model._norm_fused(3), "decode batches must take the fused normed chain"
    g = seeded(7)
    prompts = [torch.randint(1, 49151, (n,), generator=g).tolist() for n in (530, 200, 64)]
    print("fused chain: 3 requests, 6 tokens each", flush=True)
    reqs, record, alloc, executor = _run_recording(model, spec, prompts, [6, 6, 6], 512, device,
                                                   256)
    assert executor.graph_steps >= 4
    assert alloc.num_free == alloc.num_blocks
    oracle = om.OracleDecoder(weights, torch.float32)
    for r, p in zip(reqs, prompts):
        steps = record[r.request_id]
        assert [t for t, _ in steps] == r.generated_token_ids and len(steps) == 6
        _check_against_oracle(oracle, p, steps, r.request_id)


def test_smollm2_24_layers_matches_the_oracle(device) -> None:
    """The full 24-layer SmolLM2-1.7B-shaped decoder (random init on the device, INT8
    per-channel) on two short requests, decode iterations from graphs. Logits of the first token
    (from the final prefill chunk) and of every decode step match the oracle; blocks return to
    the pool; a smaller chunk size gives the same first-token logits within tolerance."""
    spec = SMOLLM2_1_7B
    model = EdgeRagDecoder(spec, 8, None, device, torch.float16)
    model.init_random(seed=11)
    g = seeded(11)
    prompts = [torch.randint(1, 49151, (n,), generator=g).tolist() for n in (300, 120)]
    print("24 layers: 2 requests (300, 120 tokens), 4 tokens each", flush=True)
    reqs, record, alloc, executor = _run_recording(model, spec, prompts, [4, 4], 512, device, 128)
    assert alloc.num_free == alloc.num_blocks
    assert executor.graph_steps >= 2
    oracle = om.OracleDecoder(model, torch.float32)
    for r, p in zip(reqs, prompts):
        steps = record[r.request_id]
        assert [t for t, _ in steps] == r.generated_token_ids and len(steps) == 4
        _check_against_oracle(oracle, p, steps, "24L " + r.request_id)
    # chunk-size invariance of the first token's logits (test_executor.py:114-130, by tolerance)
    reqs2, record2, _, _ = _run_recording(model, spec, prompts[:1], [1], 128, device, 128)
    a, b = record[reqs[0].request_id][0][1], record2[reqs2[0].request_id][0][1]
    assert float((a - b).abs().max()) <= 2e-2 * float(a.abs().max()) + 2e-2


def test_decoder_at_cfg5_lengths_through_every_decode_attention_mode(device) -> None:
    """Config 5's own lengths on two layers of the 1.7B shape (INT8 per-channel, fp16) through
    the executor with decode graphs. A 4,080-token prompt runs as eight 512-token chunks, the
    later ones over a cached prefix of up to 3,584 tokens (MFMA prefill tiles), beside seven
    shorter requests; then eight requests decode together, the long context crossing 4,096
    tokens mid-way, and the batch shrinks as requests finish. The decode graphs therefore replay
    all three attention modes: a 16-wave workgroup per (request, head), KV splits + the merge
    launch, and 8-wave workgroups over parts of each context + the merge launch. Every emitted
    token's logits are checked against OracleDecoder (fp32, teacher-forced); a 384-token chunk
    size gives the same first-token logits within tolerance (tests/test_executor.py:114-130)."""
    spec = ModelSpec("smol2", "llama", 2, 2048, 32, 32, 64, 49152, 8192, 130000.0,
                     intermediate_size=8192)
    weights = om.random_weights(spec, 13, 8, None)
    model = EdgeRagDecoder(spec, 8, None, device, torch.float16)
    model.load_quantized(weights)
    g = seeded(13)
    lens = [4080, 300, 1100, 512, 700, 256, 900, 450]
    max_new = [26, 18, 19, 20, 21, 22, 23, 24]
    prompts = [torch.randint(1, 49151, (n,), generator=g).tolist() for n in lens]
    modes: list[tuple[int, bool, int]] = []
    alloc = BlockAllocator(1024, 16)
    executor = ModelExecutor(model, spec, alloc, device, model.dtype, chunk_size=512)
    sched = Scheduler(alloc, SchedulerConfig(max_batch_size=8))
    reqs = [Request(f"r{i}", p, max_new_tokens=n) for i, (p, n) in enumerate(zip(prompts, max_new))]
    for r in reqs:
        sched.add_request(r)
    record: dict[str, list[tuple[int, torch.Tensor]]] = {r.request_id: [] for r in reqs}

    def on_step(batch, output):
        if not batch.prefill:
            modes.append(executor._fixed.mode)
        if output.tokens:
            logits = executor.last_logits.float().cpu()
            for row, (rid, token) in enumerate(output.tokens.items()):
                record[rid].append((token, logits[row]))

    print("cfg5 lengths: 8 requests, a 4,080-token prompt", flush=True)
    drive(sched, executor, on_step=on_step)
    assert alloc.num_free == alloc.num_blocks
    assert {(16, False, 0), (0, True, 0), (8, True, 16)} <= set(modes), modes
    oracle = om.OracleDecoder(weights, torch.float32)
    for r, p in zip(reqs, prompts):
        steps = record[r.request_id]
        assert [t for t, _ in steps] == r.generated_token_ids and len(steps) == r.max_new_tokens
        print(f"oracle check {r.request_id} ({len(p)} prompt tokens)", flush=True)
        _check_against_oracle(oracle, p, steps, "cfg5 " + r.request_id)
    first = {rid: steps[0][1] for rid, steps in record.items()}
    reqs2, record2, _, _ = _run_recording(model, spec, prompts[:2], [1, 1], 384, device, 512)
    for r2 in reqs2:
        a, b = first[r2.request_id], record2[r2.request_id][0][1]
        assert float((a - b).abs().max()) <= 2e-2 * float(a.abs().max()) + 2e-2


# --- the timed config-2 launch at full shape ----------------------------------------------------


def test_append_fused_on_the_full_cfg2_workload(device) -> None:
    """paged_attention_append (one launch: append fused into the decode rows) on config 2: 32
    decodes, L ~ U[256, 7472], 32/32 heads, d 64, 16,384-block pools. Pools and outputs equal
    kv_append + paged_attention bit for bit; outputs match the oracle."""
    g = seeded(2)
    lens = torch.randint(256, 7473, (32,), generator=g).tolist()
    tables, bt = _tables(lens, 16, 16384, g)
    gd = torch.Generator(device=device).manual_seed(2)
    shape = (32, 16384, 16, 64)
    kp0 = torch.randn(shape, generator=gd, device=device, dtype=torch.float16)
    vp0 = torch.randn(shape, generator=gd, device=device, dtype=torch.float16)
    q = torch.randn(32, 32, 64, generator=g).half()
    nk = torch.randn(32, 32, 64, generator=g).half()
    nv = torch.randn(32, 32, 64, generator=g).half()
    slots = np.array([tables[r][(L - 1) // 16] * 16 + (L - 1) % 16 for r, L in enumerate(lens)],
                     np.int32)
    qsl = np.arange(33, dtype=np.int32)
    plan, (slots_d,) = kernels.plan_attention(qsl, np.asarray(lens, np.int32), bt, 32, 32, 64,
                                              16, torch.float16, device, [slots])
    assert plan.decode_only
    qd, nkd, nvd = q.to(device), nk.to(device), nv.to(device)
    kp1, vp1 = kp0.clone(), vp0.clone()
    kernels.kv_append(nkd, nvd, slots_d, kp1, vp1)
    ref = kernels.paged_attention(qd, kp1, vp1, plan, 0.125, overlap=False)
    kp2, vp2 = kp0, vp0  # the fused launch appends in place
    got = kernels.paged_attention_append(nkd, nvd, slots_d, qd, kp2, vp2, plan, 0.125)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(kp2, kp1) and torch.equal(vp2, vp1)
    del kp1, vp1
    expected = oa.ragged_reference(q, kp2.cpu(), vp2.cpu(), qsl.tolist(), lens, tables, 0.125)
    torch.testing.assert_close(got.float().cpu(), expected, **FP16_TOL)


# --- block sizes other than 16 ------------------------------------------------------------------


@pytest.mark.parametrize("bs", [4, 8, 12, 32, 64])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_attention_at_other_block_sizes(device, bs, dtype) -> None:
    """Mixed prefill slices + decodes over pools of block size 4 / 8 / 12 / 32 / 64 with poisoned
    slack: the fast decode kernel (block size a multiple of its 8 tokens per load), the general
    row kernel (12, and fp32), and the MFMA prefill tiles (powers of two >= 4, fp16)."""
    g = seeded(bs * 7 + (dtype == torch.float16))
    lens = [700, 97, 1300 + 130, 33, 2900, 5]
    q_lens = [300, 1, 130, 1, 1, 5]
    n_q, n_kv, d = 8, 4, 64
    NB = sum(math.ceil(L / bs) for L in lens) + 4
    kp = torch.randn((n_kv, NB, bs, d), generator=g).to(dtype)
    vp = torch.randn((n_kv, NB, bs, d), generator=g).to(dtype)
    tables, bt = _tables(lens, bs, NB, g)
    for L, t in zip(lens, tables):
        if L % bs:
            kp[:, t[-1], L % bs :] = 1e4
            vp[:, t[-1], L % bs :] = 1e4
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    q = torch.randn(int(qsl[-1]), n_q, d, generator=g).to(dtype)
    got = ragged_paged_attention(q.to(device), kp.to(device), vp.to(device), qsl,
                                 np.asarray(lens, np.int32), bt, 0.125).cpu()
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, 0.125)
    tol = FP32_TOL if dtype == torch.float32 else FP16_TOL
    torch.testing.assert_close(got.float(), expected, **tol)
    # float64 pin of one decode row
    r, h = 4, 3
    k = op.gather_pool(kp.double(), tables[r], lens[r])[h // 2]
    v = op.gather_pool(vp.double(), tables[r], lens[r])[h // 2]
    ref64 = oa.attention_f64(q[qsl[r] : qsl[r + 1], h], k, v, lens[r] - 1, 0.125)
    torch.testing.assert_close(got[qsl[r] : qsl[r + 1], h].double(), ref64,
                               **{k_: v_ * 2 for k_, v_ in tol.items()})
