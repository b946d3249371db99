"""Paged attention on the GPU against the oracle.

Cases restate the reference's own tests (tests/test_fused_attention.py) and its GPU gate
(scripts/colab_fused_attention.py:62, :132-133, :254), then widen to the ragged decode +
chunked-prefill batches of BASELINE configs 1-3.

Tolerances, written where they are used:
* fp32 pools: 1e-5 (test_fused_attention.py:91);
* fp16 pools: atol 2e-3 / rtol 1e-2 (north_star; colab_fused_attention.py:254).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from edgerag_amd import kernels
from edgerag_amd.cache.fused import fused_paged_attention, ragged_paged_attention
from oracle import attention as oa
from oracle import paged as op
from tests.conftest import seeded

pytestmark = pytest.mark.gpu

BLOCK_SIZE = 16
FP32_TOL = dict(rtol=1e-5, atol=1e-5)
FP16_TOL = dict(rtol=1e-2, atol=2e-3)


def _pool(n_kv_heads, num_blocks, head_dim, dtype, g):
    shape = (n_kv_heads, num_blocks, BLOCK_SIZE, head_dim)
    return torch.randn(shape, generator=g).to(dtype), torch.randn(shape, generator=g).to(dtype)


# --- fused_paged_attention: the reference's own cases ------------------------------------------


@pytest.mark.parametrize(
    "seq_len", [1, 2, 15, 16, 17, 31, 32, 33, 47, 48, 49, 63, 64, 65, 100, 127, 128, 129]
)
def test_decode_matches_reference_across_block_boundaries(device, seq_len) -> None:
    """test_fused_attention.py:71-91 (head_dim 8, fp32, 1e-5)."""
    g = seeded(seq_len)
    n_kv, d = 4, 8
    nb = math.ceil(seq_len / BLOCK_SIZE)
    kp, vp = _pool(n_kv, nb + 3, d, torch.float32, g)
    ids = torch.randperm(nb + 3, generator=g)[:nb]
    q = torch.randn(1, n_kv, 1, d, generator=g)
    scale = d**-0.5
    expected = oa.sdpa_over_gather(q, kp, vp, ids, seq_len, scale, 1)
    spec = oa.paged_attention_reference(q, kp, vp, ids, seq_len, scale, 1)
    torch.testing.assert_close(spec, expected, **FP32_TOL)
    got = fused_paged_attention(q.to(device), kp.to(device), vp.to(device), ids.to(device),
                                seq_len, scale)
    assert got.shape == (1, 1, n_kv, d) and got.dtype == torch.float32
    torch.testing.assert_close(got.cpu(), spec, **FP32_TOL)


def test_unwritten_tail_of_final_block_is_never_attended(device) -> None:
    """test_fused_attention.py:94-116: poison the slack with 1e4."""
    g = seeded(17)
    kp, vp = _pool(2, 4, 8, torch.float32, g)
    ids = torch.tensor([0, 1])
    q = torch.randn(1, 2, 1, 8, generator=g)
    args = (ids.to(device), 17, 8**-0.5)
    clean = fused_paged_attention(q.to(device), kp.to(device), vp.to(device), *args)
    kp[:, 1, 1:] = 1e4
    vp[:, 1, 1:] = 1e4
    poisoned = fused_paged_attention(q.to(device), kp.to(device), vp.to(device), *args)
    torch.testing.assert_close(poisoned, clean, rtol=1e-6, atol=1e-6)


def test_blocks_past_the_written_region_are_not_read(device) -> None:
    """test_fused_attention.py:119-131."""
    g = seeded(20)
    kp, vp = _pool(2, 6, 8, torch.float32, g)
    kp[:, 2:] = 1e4
    vp[:, 2:] = 1e4
    q = torch.randn(1, 2, 1, 8, generator=g).to(device)
    kp, vp = kp.to(device), vp.to(device)
    a = fused_paged_attention(q, kp, vp, torch.tensor([0, 1], device=device), 20, 8**-0.5)
    b = fused_paged_attention(q, kp, vp, torch.tensor([0, 1, 2, 3], device=device), 20, 8**-0.5)
    torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("n_rep", [1, 2, 3, 4])
def test_grouped_query_heads_map_consecutively(device, n_rep) -> None:
    """test_fused_attention.py:134-154: kv_head = q_head // n_rep."""
    g = seeded(40 + n_rep)
    n_kv = 3
    kp, vp = _pool(n_kv, 5, 8, torch.float32, g)
    ids = torch.tensor([0, 1, 2])
    q = torch.randn(1, n_kv * n_rep, 1, 8, generator=g)
    expected = oa.sdpa_over_gather(q, kp, vp, ids, 40, 8**-0.5, n_rep)
    got = fused_paged_attention(q.to(device), kp.to(device), vp.to(device), ids.to(device), 40,
                                8**-0.5, n_rep)
    torch.testing.assert_close(got.cpu(), expected, **FP32_TOL)


def test_scattered_block_table(device) -> None:
    """test_fused_attention.py:157-169."""
    g = seeded(48)
    kp, vp = _pool(2, 8, 8, torch.float32, g)
    ids = torch.tensor([7, 2, 5])
    q = torch.randn(1, 2, 1, 8, generator=g)
    expected = oa.sdpa_over_gather(q, kp, vp, ids, 48, 8**-0.5, 1)
    got = fused_paged_attention(q.to(device), kp.to(device), vp.to(device), ids.to(device), 48,
                                8**-0.5)
    torch.testing.assert_close(got.cpu(), expected, **FP32_TOL)


def test_scores_that_would_overflow_a_naive_softmax_stay_finite(device) -> None:
    """test_fused_attention.py:175-190."""
    g = seeded(33)
    kp, vp = _pool(2, 4, 8, torch.float32, g)
    kp *= 200.0
    q = torch.randn(1, 2, 1, 8, generator=g) * 200.0
    ids = torch.tensor([0, 1, 2])
    got = fused_paged_attention(q.to(device), kp.to(device), vp.to(device), ids.to(device), 33,
                                8**-0.5)
    assert torch.isfinite(got).all()
    expected = oa.paged_attention_reference(q, kp, vp, ids, 33, 8**-0.5)
    torch.testing.assert_close(got.cpu(), expected, rtol=1e-4, atol=1e-4)


def test_empty_sequence_returns_zeros(device) -> None:
    """test_fused_attention.py:193-201."""
    g = seeded(0)
    kp, vp = _pool(2, 2, 8, torch.float32, g)
    out = fused_paged_attention(torch.randn(1, 2, 1, 8).to(device), kp.to(device), vp.to(device),
                                torch.tensor([0], device=device), 0, 8**-0.5)
    assert torch.isfinite(out).all() and torch.count_nonzero(out) == 0


def test_guards(device) -> None:
    """test_fused_attention.py:207-223: prefill refused; head mismatch refused."""
    g = seeded(1)
    kp, vp = _pool(2, 4, 8, torch.float32, g)
    kp, vp = kp.to(device), vp.to(device)
    with pytest.raises(ValueError, match="decode path"):
        fused_paged_attention(torch.randn(1, 2, 7, 8, device=device), kp, vp,
                              torch.tensor([0], device=device), 16, 8**-0.5)
    with pytest.raises(ValueError, match="query heads"):
        fused_paged_attention(torch.randn(1, 6, 1, 8, device=device), kp, vp,
                              torch.tensor([0], device=device), 16, 8**-0.5, n_rep=1)


@pytest.mark.parametrize(
    "seq_len", [1, 2, 15, 16, 17, 31, 32, 33, 127, 128, 129, 511, 512, 513, 6758, 6759]
)
def test_fp16_gate_lengths_with_poisoned_slack(device, seq_len) -> None:
    """colab_fused_attention.py:62 gate lengths, slack poisoned with 1e4 (:132-133), 2e-3."""
    g = seeded(seq_len + 1000)
    n_kv, d = 32, 64
    nb = math.ceil(seq_len / BLOCK_SIZE)
    kp, vp = _pool(n_kv, nb + 2, d, torch.float16, g)
    ids = torch.randperm(nb + 2, generator=g)[:nb]
    last, used = int(ids[-1]), seq_len - (nb - 1) * BLOCK_SIZE
    kp[:, last, used:] = 1e4
    vp[:, last, used:] = 1e4
    q = torch.randn(1, n_kv, 1, d, generator=g).half()
    expected = oa.paged_attention_reference(q.float(), kp.float(), vp.float(), ids, seq_len,
                                            d**-0.5)
    got = fused_paged_attention(q.to(device), kp.to(device), vp.to(device), ids.to(device),
                                seq_len, d**-0.5)
    assert got.dtype == torch.float16
    torch.testing.assert_close(got.float().cpu(), expected, **FP16_TOL)


# --- ragged batches ----------------------------------------------------------------------------


def _ragged_case(lens, q_lens, n_q, n_kv, d, dtype, seed, pool_blocks=None, poison=True):
    """Seeded ragged batch: pools, disjoint tables from one permutation, packed queries."""
    g = seeded(seed)
    nbs = [math.ceil(L / BLOCK_SIZE) for L in lens]
    NB = pool_blocks or (sum(nbs) + 4)
    kp, vp = _pool(n_kv, NB, d, dtype, g)
    perm = torch.randperm(NB, generator=g).tolist()
    tables, at = [], 0
    for nb in nbs:
        tables.append(perm[at : at + nb])
        at += nb
    if poison:
        for L, t in zip(lens, tables):
            if t and L % BLOCK_SIZE:
                kp[:, t[-1], L % BLOCK_SIZE :] = 1e4
                vp[:, t[-1], L % BLOCK_SIZE :] = 1e4
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    q = torch.randn(int(qsl[-1]), n_q, d, generator=g).to(dtype)
    maxb = max(nbs + [1])
    bt = np.full((len(lens), maxb), -1, np.int32)
    for r, t in enumerate(tables):
        bt[r, : len(t)] = t
    return kp, vp, tables, qsl, q, bt


def _run_ragged(device, kp, vp, qsl, lens, bt, q, scale):
    return ragged_paged_attention(
        q.to(device), kp.to(device), vp.to(device), qsl, np.asarray(lens, np.int32), bt, scale
    ).cpu()


def test_cfg1_gqa_decode_batch_fp32(device) -> None:
    """lengths [37,128,300,511], 9/3 heads, d 64, pool 64, fp32, 1e-5."""
    lens = [37, 128, 300, 511]
    kp, vp, tables, qsl, q, bt = _ragged_case(lens, [1] * 4, 9, 3, 64, torch.float32, 11,
                                              pool_blocks=64)
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, 0.125)
    got = _run_ragged(device, kp, vp, qsl, lens, bt, q, 0.125)
    torch.testing.assert_close(got, expected, **FP32_TOL)
    # and against the blockwise spec per request
    for r, L in enumerate(lens):
        spec = oa.paged_attention_reference(
            q[r][None, :, None], kp, vp, torch.tensor(tables[r]), L, 0.125, 3
        )
        torch.testing.assert_close(got[r], spec[0, 0], **FP32_TOL)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_mixed_prefill_chunks_and_decodes(device, dtype) -> None:
    """A cfg3-shaped batch, scaled down: prefill slices (causal + prefix) beside decodes."""
    lens = [40, 64 + 37, 300, 17, 1000, 5]
    q_lens = [40, 37, 1, 1, 129, 5]  # chunk at offset 0, chunk at offset 64, decodes, ...
    tol = FP32_TOL if dtype == torch.float32 else FP16_TOL
    kp, vp, tables, qsl, q, bt = _ragged_case(lens, q_lens, 8, 4, 64, dtype, 77)
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, 0.125)
    got = _run_ragged(device, kp, vp, qsl, lens, bt, q, 0.125)
    torch.testing.assert_close(got.float(), expected, **tol)
    # float64 textbook pin for one head of the offset chunk
    r, h = 1, 5
    k = op.gather_pool(kp.float(), tables[r], lens[r])[h // 2]
    v = op.gather_pool(vp.float(), tables[r], lens[r])[h // 2]
    ref64 = oa.attention_f64(q[qsl[r] : qsl[r + 1], h], k, v, lens[r] - q_lens[r], 0.125)
    torch.testing.assert_close(got[qsl[r] : qsl[r + 1], h].double(), ref64, **{
        k_: v_ * 2 for k_, v_ in tol.items()})


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [16, 32, 256])
def test_mixed_batch_other_head_dims(device, dtype, d) -> None:
    """The same mixed batch at the other head dims the kernels instantiate (the row kernels take
    the prefill slices there), in fp16 and bf16; one head of the offset chunk against the float64
    textbook softmax as well."""
    lens = [40, 64 + 37, 300, 17, 1000, 5]
    q_lens = [40, 37, 1, 1, 129, 5]
    scale = d**-0.5
    # bf16 rounds q, K, V and the output to 8 significant bits.
    tol = FP16_TOL if dtype == torch.float16 else dict(rtol=2e-2, atol=1e-2)
    kp, vp, tables, qsl, q, bt = _ragged_case(lens, q_lens, 8, 4, d, dtype, 91 + d)
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, scale)
    got = _run_ragged(device, kp, vp, qsl, lens, bt, q, scale)
    assert got.dtype == dtype
    torch.testing.assert_close(got.float(), expected, **tol)
    r, h = 1, 5
    k = op.gather_pool(kp.float(), tables[r], lens[r])[h // 2]
    v = op.gather_pool(vp.float(), tables[r], lens[r])[h // 2]
    ref64 = oa.attention_f64(q[qsl[r] : qsl[r + 1], h].float(), k, v, lens[r] - q_lens[r], scale)
    torch.testing.assert_close(got[qsl[r] : qsl[r + 1], h].double(), ref64,
                               **{k_: v_ * 2 for k_, v_ in tol.items()})


def test_chunked_prefill_equals_single_shot(device) -> None:
    """test_batched.py:80-119 restated: 3 chunks over the same pool == 1 chunk."""
    L, d = 300, 64
    kp, vp, tables, _, q, bt = _ragged_case([L], [L], 4, 4, d, torch.float32, 5)
    one = _run_ragged(device, kp, vp, np.array([0, L], np.int32), [L], bt, q, 0.125)
    parts = []
    for start, end in ((0, 128), (128, 256), (256, 300)):
        parts.append(_run_ragged(device, kp, vp, np.array([0, end - start], np.int32), [end], bt,
                                 q[start:end], 0.125))
    torch.testing.assert_close(torch.cat(parts), one, rtol=5e-5 * 3, atol=5e-5 * 3)


def test_single_chunk_without_prefix_equals_causal_sdpa(device) -> None:
    """Special case: past = 0 reduces to SDPA(is_causal=True), a library routine."""
    L = 257
    kp, vp, tables, qsl, q, bt = _ragged_case([L], [L], 4, 2, 64, torch.float32, 6)
    k = op.gather_pool(kp, tables[0], L).repeat_interleave(2, dim=0)
    v = op.gather_pool(vp, tables[0], L).repeat_interleave(2, dim=0)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(0, 1), k, v, is_causal=True, scale=0.125
    ).transpose(0, 1)
    got = _run_ragged(device, kp, vp, qsl, [L], bt, q, 0.125)
    torch.testing.assert_close(got, ref, **FP32_TOL)


def test_zero_query_requests_and_empty_batch(device) -> None:
    lens = [33, 50, 20]
    kp, vp, tables, qsl, q, bt = _ragged_case(lens, [1, 0, 2], 4, 4, 64, torch.float32, 8)
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, 0.125)
    got = _run_ragged(device, kp, vp, qsl, lens, bt, q, 0.125)
    torch.testing.assert_close(got, expected, **FP32_TOL)


def test_repeated_launches_with_a_shared_workspace_agree(device) -> None:
    """Split partials live in a workspace reused across launches and plans: back-to-back
    launches (with another plan's launch in between) must agree bit for bit."""
    lens = [2000, 1500, 3000, 700]
    kp, vp, tables, qsl, q, bt = _ragged_case(lens, [1] * 4, 8, 4, 64, torch.float16, 12)
    kd, vd, qd = kp.to(device), vp.to(device), q.to(device)
    plan, _ = kernels.plan_attention(qsl, np.asarray(lens, np.int32), bt, 8, 4, 64, BLOCK_SIZE,
                                     torch.float16, device, split_rows=True)
    assert int(plan.plan_host[6]) > 0, "the case must exercise split merging (partials)"
    other, _ = kernels.plan_attention(qsl[:3], np.asarray(lens[:2], np.int32), bt[:2], 8, 4, 64,
                                      BLOCK_SIZE, torch.float16, device, split_rows=True)
    outs = []
    for _ in range(3):
        outs.append(kernels.paged_attention(qd, kd, vd, plan, 0.125).clone())
        kernels.paged_attention(qd[:2], kd, vd, other, 0.125)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, 0.125)
    torch.testing.assert_close(outs[0].float().cpu(), expected, **FP16_TOL)


def test_graph_replays_match_eager_with_split_merge(device) -> None:
    """The decode kernel and the split merge captured in a HIP graph, replayed several times with
    eager launches and synchronisations in between, reproduce the eager result on every replay."""
    lens = [3000, 257, 4100, 1800, 900, 6000]
    kp, vp, tables, qsl, q, bt = _ragged_case(lens, [1] * 6, 8, 8, 64, torch.float16, 21)
    kd, vd, qd = kp.to(device), vp.to(device), q.to(device)
    plan, _ = kernels.plan_attention(qsl, np.asarray(lens, np.int32), bt, 8, 8, 64, BLOCK_SIZE,
                                     torch.float16, device, split_rows=True)
    assert int(plan.plan_host[6]) > 0 and int(plan.plan_host[16]) > 0
    eager = kernels.paged_attention(qd, kd, vd, plan, 0.125).clone()
    out = torch.empty_like(qd)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kernels.paged_attention(qd, kd, vd, plan, 0.125, out=out)
    for _ in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        again = kernels.paged_attention(qd, kd, vd, plan, 0.125)
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, 0.125)
    torch.testing.assert_close(eager.float().cpu(), expected, **FP16_TOL)


def test_plans_of_different_sizes_share_one_workspace(device) -> None:
    """Plans of different sizes (different partial layouts) alternate on one shared workspace."""
    small = [2600, 3100]
    large = [700 + 137 * i for i in range(40)]
    cases = []
    for lens, seed in ((small, 31), (large, 32)):
        kp, vp, tables, qsl, q, bt = _ragged_case(lens, [1] * len(lens), 8, 8, 64, torch.float16,
                                                  seed)
        plan, _ = kernels.plan_attention(qsl, np.asarray(lens, np.int32), bt, 8, 8, 64,
                                         BLOCK_SIZE, torch.float16, device, split_rows=True)
        assert int(plan.plan_host[6]) > 0
        expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, 0.125)
        cases.append((kp.to(device), vp.to(device), q.to(device), plan, expected))
    for _ in range(2):
        for kd, vd, qd, plan, expected in cases:
            got = kernels.paged_attention(qd, kd, vd, plan, 0.125)
            torch.testing.assert_close(got.float().cpu(), expected, **FP16_TOL)


def test_plan_rejects_more_queries_than_context(device) -> None:
    kp, vp, tables, qsl, q, bt = _ragged_case([10], [10], 4, 4, 64, torch.float32, 8)
    with pytest.raises(kernels._lib.EdgeragError, match="queries but context"):
        _run_ragged(device, kp, vp, np.array([0, 10], np.int32), [9], bt, q, 0.125)


@pytest.mark.parametrize("n_q,n_kv", [(32, 32), (9, 3), (8, 1)])
def test_cfg3_shape_mixed_batch_fp16(device, n_q, n_kv) -> None:
    """prefill slices of 512 at offsets 0 / 3584 / 6656 beside 24 decodes
    with L ~ U[512, 7472]; fp16, d 64 (the MFMA tile path), plus GQA groupings."""
    g = seeded(3)
    dec = torch.randint(512, 7473, (24,), generator=g).tolist()
    lens = [512, 3584 + 512, 6656 + 512] + dec
    q_lens = [512, 512, 512] + [1] * 24
    kp, vp, tables, qsl, q, bt = _ragged_case(lens, q_lens, n_q, n_kv, 64, torch.float16, 31)
    got = _run_ragged(device, kp, vp, qsl, lens, bt, q, 0.125)
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, 0.125)
    torch.testing.assert_close(got.float(), expected, **FP16_TOL)


@pytest.mark.parametrize("c,past", [(1, 0), (7, 0), (64, 0), (65, 13), (130, 200), (512, 3584)])
def test_fp16_prefill_chunk_edges(device, c, past) -> None:
    """Tile edges: partial 128-row tiles, chunks shorter than one 64-key tile, ragged prefixes."""
    L = past + c
    kp, vp, tables, qsl, q, bt = _ragged_case([L], [c], 4, 4, 64, torch.float16, c + past)
    got = _run_ragged(device, kp, vp, qsl, [L], bt, q, 0.125)
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), [L], tables, 0.125)
    torch.testing.assert_close(got.float(), expected, **FP16_TOL)


def test_cfg2_shape_decode_batch_fp16(device) -> None:
    """BASELINE config 2 at full shape: 32 decodes, L ~ U[256, 7472], 32/32 heads, d 64,
    16,384-block pool (1 GiB per pool), seeded-shuffled tables."""
    g = seeded(2)
    lens = torch.randint(256, 7473, (32,), generator=g).tolist()
    nbs = [math.ceil(L / BLOCK_SIZE) for L in lens]
    perm = torch.randperm(16384, generator=g).tolist()
    tables, at = [], 0
    for nb in nbs:
        tables.append(perm[at : at + nb])
        at += nb
    gd = torch.Generator(device=device).manual_seed(2)
    shape = (32, 16384, BLOCK_SIZE, 64)
    kp_d = torch.randn(shape, generator=gd, device=device, dtype=torch.float16)
    vp_d = torch.randn(shape, generator=gd, device=device, dtype=torch.float16)
    q = torch.randn(32, 32, 64, generator=g).half()
    qsl = np.arange(33, dtype=np.int32)
    bt = np.full((32, max(nbs)), -1, np.int32)
    for r, t in enumerate(tables):
        bt[r, : len(t)] = t
    got = ragged_paged_attention(q.to(device), kp_d, vp_d, qsl, np.asarray(lens, np.int32), bt,
                                 0.125).cpu()
    expected = oa.ragged_reference(q, kp_d.cpu(), vp_d.cpu(), qsl.tolist(), lens, tables, 0.125)
    torch.testing.assert_close(got.float(), expected, **FP16_TOL)


@pytest.mark.parametrize("q_len", [1, 200])
def test_invalid_block_ids_mask_their_keys(device, q_len) -> None:
    """A block id outside [0, num_blocks) (never produced by the allocator) hides its 16 keys
    instead of reading out of bounds; the decode row kernel (q_len 1) and the MFMA prefill tiles
    (q_len 200) agree with a float64 softmax that excludes exactly those keys."""
    L, n_q, n_kv, d = 600, 8, 4, 64
    kp, vp, tables, qsl, q, bt = _ragged_case([L], [q_len], n_q, n_kv, d, torch.float16, 91,
                                              poison=False)
    NB = kp.shape[1]
    bt[0, 5] = -1
    bt[0, 20] = NB + 3
    bad = torch.zeros(L, dtype=torch.bool)
    bad[5 * BLOCK_SIZE : 6 * BLOCK_SIZE] = True
    bad[20 * BLOCK_SIZE : 21 * BLOCK_SIZE] = True
    got = _run_ragged(device, kp, vp, qsl, [L], bt, q, 0.125)
    k = op.gather_pool(kp.double(), tables[0], L)  # (n_kv, L, d), real contents of every block
    v = op.gather_pool(vp.double(), tables[0], L)
    pos = torch.arange(L)
    for h in range(n_q):
        qh = q[:, h].double()  # (q_len, d)
        s = qh @ k[h // 2].T * 0.125
        visible = (pos[None, :] <= (L - q_len + torch.arange(q_len))[:, None]) & ~bad[None, :]
        s = s.masked_fill(~visible, float("-inf"))
        ref = torch.softmax(s, dim=-1) @ v[h // 2]
        torch.testing.assert_close(got[:, h].double(), ref, rtol=1e-2, atol=2e-3)


@pytest.mark.parametrize("dtype,n_q,n_kv,d,q_lens", [
    (torch.float16, 32, 32, 64, None),     # config-2-shaped decode batch
    (torch.float32, 8, 2, 64, None),       # GQA, fp32
    (torch.bfloat16, 8, 2, 128, None),     # GQA, head_dim 128
    (torch.float16, 8, 4, 64, "multi"),    # 2-token rows (2 * n_rep <= 8 query vectors)
    (torch.float16, 8, 4, 64, "mixed"),    # a prefill slice in the batch: two launches
])
def test_append_fused_into_attention_equals_append_then_attention(device, dtype, n_q, n_kv, d,
                                                                  q_lens) -> None:
    """paged_attention_append == kv_append followed by paged_attention, bit for bit: outputs,
    key pool and value pool. Decode batches run as one launch (the new positions are read from
    the new rows and written to their slots by the waves that reach them); a batch with a
    prefill slice takes the two-launch path through the same entry."""
    g = seeded(len(str(q_lens)) + d + n_q)
    lens = [int(x) for x in torch.randint(1, 1500, (24,), generator=g)]
    if q_lens is None:
        q_lens = [1] * len(lens)
    elif q_lens == "multi":
        q_lens = [min(2, L) for L in lens]
    else:
        lens[3], lens[7] = 700, 200
        q_lens = [1] * len(lens)
        q_lens[3] = 200  # a 200-token chunk after a 500-token prefix
    kp, vp, tables, qsl, q, bt = _ragged_case(lens, q_lens, n_q, n_kv, d, dtype, 31,
                                              poison=False)
    T = int(qsl[-1])
    nk = torch.randn(T, n_kv, d, generator=g).to(dtype)
    nv = torch.randn(T, n_kv, d, generator=g).to(dtype)
    slots = []
    for r, (L, c) in enumerate(zip(lens, q_lens)):
        for pos in range(L - c, L):
            slots.append(tables[r][pos // BLOCK_SIZE] * BLOCK_SIZE + pos % BLOCK_SIZE)
    slots = torch.tensor(slots, dtype=torch.int32)
    plan, (slots_d,) = kernels.plan_attention(qsl, np.asarray(lens, np.int32), bt, n_q, n_kv, d,
                                              BLOCK_SIZE, dtype, device, [slots.numpy()])
    scale = d ** -0.5
    qd, nkd, nvd = q.to(device), nk.to(device), nv.to(device)
    kp1, vp1 = kp.to(device), vp.to(device)
    kernels.kv_append(nkd, nvd, slots_d, kp1, vp1)
    ref = kernels.paged_attention(qd, kp1, vp1, plan, scale, overlap=False)
    kp2, vp2 = kp.to(device), vp.to(device)
    got = kernels.paged_attention_append(nkd, nvd, slots_d, qd, kp2, vp2, plan, scale)
    assert torch.equal(got, ref)
    assert torch.equal(kp2, kp1) and torch.equal(vp2, vp1)
    # and the result is attention over the appended pools (float64 pin on one request)
    r = 5
    kh = op.gather_pool(kp1.cpu().float(), tables[r], lens[r])[0]
    vh = op.gather_pool(vp1.cpu().float(), tables[r], lens[r])[0]
    ref64 = oa.attention_f64(q[qsl[r] : qsl[r + 1], 0], kh, vh, lens[r] - q_lens[r], scale)
    tol = FP32_TOL if dtype == torch.float32 else {k_: v_ * 4 for k_, v_ in FP16_TOL.items()}
    torch.testing.assert_close(got[qsl[r] : qsl[r + 1], 0].cpu().double(), ref64, **tol)


@pytest.mark.parametrize("dtype,n_q,n_kv,d,dec", [
    (torch.float16, 8, 4, 64, [300, 17, 1000, 5]),  # MFMA tiles beside decode rows
    (torch.float16, 9, 3, 64, None),                 # config 3 lengths, GQA
    (torch.float32, 8, 4, 64, [300, 17, 1000, 5]),  # tiles on the row kernel
    (torch.bfloat16, 4, 2, 128, [900, 33]),
])
def test_two_stream_overlap_equals_one_stream(device, dtype, n_q, n_kv, d, dec) -> None:
    """Decode rows on a second stream beside the prefill tiles (planned when both are heavy;
    forced here with EDGERAG_PLAN_OVERLAP) give the one-stream results of the same plan bit for
    bit, through paged_attention and paged_attention_append alike."""
    g = seeded(d + n_q + len(dec or []))
    if dec is None:
        dec = torch.randint(512, 7473, (24,), generator=g).tolist()
        lens, q_lens = [512, 3584 + 512, 6656 + 512] + dec, [512, 512, 512] + [1] * len(dec)
    else:
        lens, q_lens = [40, 64 + 37, 129 + 200] + dec, [40, 37, 129] + [1] * len(dec)
    kp, vp, tables, qsl, q, bt = _ragged_case(lens, q_lens, n_q, n_kv, d, dtype, 53,
                                              poison=False)
    T = int(qsl[-1])
    nk = torch.randn(T, n_kv, d, generator=g).to(dtype)
    nv = torch.randn(T, n_kv, d, generator=g).to(dtype)
    slots = np.array([tables[r][p // BLOCK_SIZE] * BLOCK_SIZE + p % BLOCK_SIZE
                      for r, (L, c) in enumerate(zip(lens, q_lens)) for p in range(L - c, L)],
                     np.int32)
    plan, (slots_d,) = kernels.plan_attention(qsl, np.asarray(lens, np.int32), bt, n_q, n_kv, d,
                                              BLOCK_SIZE, dtype, device, [slots],
                                              force_overlap=True)
    assert plan.overlap_rows
    scale = d ** -0.5
    qd, kpd, vpd = q.to(device), kp.to(device), vp.to(device)
    one = kernels.paged_attention(qd, kpd, vpd, plan, scale, overlap=False)
    two = kernels.paged_attention(qd, kpd, vpd, plan, scale, overlap=True)
    torch.cuda.synchronize()
    assert torch.equal(two, one)
    tol = FP32_TOL if dtype == torch.float32 else dict(rtol=2e-2, atol=1e-2)
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, scale)
    torch.testing.assert_close(two.cpu().float(), expected, **tol)
    nkd, nvd = nk.to(device), nv.to(device)
    kp1, vp1 = kp.to(device), vp.to(device)
    kernels.kv_append(nkd, nvd, slots_d, kp1, vp1)
    ref = kernels.paged_attention(qd, kp1, vp1, plan, scale, overlap=False)
    got = kernels.paged_attention_append(nkd, nvd, slots_d, qd, kpd, vpd, plan, scale,
                                         overlap=True)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(kpd, kp1) and torch.equal(vpd, vp1)


def test_one_and_two_stream_plans_agree(device) -> None:
    """A serving-shaped batch (a 512-token chunk after a 3,000-token prefix beside 7 decodes) is
    planned for one stream by default (128 tiles split toward 512 items, rows sized to run
    alone) and for two with EDGERAG_PLAN_OVERLAP (256 tile items, tiles at one workgroup per
    CU). Both plans give the oracle's attention; they differ only in summation order."""
    dec = [3000, 2500, 4000, 1200, 3300, 700, 3900]
    lens, q_lens = [3512] + dec, [512] + [1] * len(dec)
    kp, vp, tables, qsl, q, bt = _ragged_case(lens, q_lens, 32, 32, 64, torch.float16, 61)
    ctx = np.asarray(lens, np.int32)
    one, _ = kernels.plan_attention(qsl, ctx, bt, 32, 32, 64, BLOCK_SIZE, torch.float16, device)
    two, _ = kernels.plan_attention(qsl, ctx, bt, 32, 32, 64, BLOCK_SIZE, torch.float16, device,
                                    force_overlap=True)
    assert not one.overlap_rows and two.overlap_rows
    assert one.n_items - int(one.plan_host[13]) >= 512 > two.n_items - int(two.plan_host[13])
    qd, kpd, vpd = q.to(device), kp.to(device), vp.to(device)
    got1 = kernels.paged_attention(qd, kpd, vpd, one, 0.125).cpu()
    got2 = kernels.paged_attention(qd, kpd, vpd, two, 0.125).cpu()
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, 0.125)
    torch.testing.assert_close(got1.float(), expected, **FP16_TOL)
    torch.testing.assert_close(got2.float(), expected, **FP16_TOL)
    torch.testing.assert_close(got1, got2, **FP16_TOL)


@pytest.mark.parametrize("lens,n_q,n_kv", [
    ([256], 32, 32), ([1000], 32, 32), ([3000], 32, 32), ([4097], 32, 32), ([6758], 32, 32),
    ([7472], 32, 32), ([256, 7472], 32, 32), ([3000, 4100], 32, 32), ([7472, 7000], 32, 32),
    ([5000], 9, 3), ([2500, 700], 8, 1),
])
def test_few_decodes_as_context_parts_fp16(device, lens, n_q, n_kv) -> None:
    """Batches of one or two decodes (fewer row workgroups than CUs): every context cut into
    parts of 8-wave workgroups merged by the combine launch, slack poisoned with 1e4; against
    the oracle at the fp16 gate tolerance. The append fused into the same launch writes the pools
    exactly as kv_append does."""
    d = 64
    q_lens = [1] * len(lens)
    kp, vp, tables, qsl, q, bt = _ragged_case(lens, q_lens, n_q, n_kv, d, torch.float16,
                                              sum(lens) + n_q)
    plan_host, _ = kernels.make_plan_host(qsl, np.asarray(lens, np.int32), n_q, n_kv, d,
                                          BLOCK_SIZE, bt.shape[1], torch.float16)
    assert int(plan_host[19]) == 8, "expected workgroups over parts of the contexts"
    # Parts (of >= 8 x 32 tokens, 8 x 16 when no context passes 2,048) in fixed slots: every
    # token has a merge row, split or not; nothing to merge when no context is cut.
    min_part = 128 if max(lens) <= 2048 else 256
    split = any(L > min_part for L in lens)
    assert int(plan_host[21]) == ((16 if n_kv == 32 else 32) if split else 0)
    assert int(plan_host[16]) == (len(lens) if split else 0)
    got = _run_ragged(device, kp, vp, qsl, lens, bt, q, d**-0.5)
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, d**-0.5)
    torch.testing.assert_close(got.float(), expected, **FP16_TOL)
    # The append fused into the parts' launch: the step's own token read from the new rows.
    g = seeded(len(lens) + 7)
    nk = torch.randn(len(lens), n_kv, d, generator=g).half()
    nv = torch.randn(len(lens), n_kv, d, generator=g).half()
    slots = torch.tensor([tables[r][(L - 1) // BLOCK_SIZE] * BLOCK_SIZE + (L - 1) % BLOCK_SIZE
                          for r, L in enumerate(lens)], dtype=torch.int32)
    plan, (slots_d,) = kernels.plan_attention(qsl, np.asarray(lens, np.int32), bt, n_q, n_kv, d,
                                              BLOCK_SIZE, torch.float16, device, [slots.numpy()])
    qd, nkd, nvd = q.to(device), nk.to(device), nv.to(device)
    kp1, vp1 = kp.to(device), vp.to(device)
    kernels.kv_append(nkd, nvd, slots_d, kp1, vp1)
    ref = kernels.paged_attention(qd, kp1, vp1, plan, d**-0.5)
    kp2, vp2 = kp.to(device), vp.to(device)
    fused = kernels.paged_attention_append(nkd, nvd, slots_d, qd, kp2, vp2, plan, d**-0.5)
    assert torch.equal(fused, ref)
    assert torch.equal(kp2, kp1) and torch.equal(vp2, vp1)


@pytest.mark.parametrize("c,past,q_lens_kind", [(512, 3584, "prefill"), (200, 900, "prefill"),
                                                (1, 4000, "decode")])
def test_large_scores_and_attention_sinks_fp16(device, c, past, q_lens_kind) -> None:
    """Scores far from the unit-variance regime: Q and K scaled 8x (scores of tens of nats) and
    four attention-sink keys aligned with every query; prefill MFMA tiles and decode rows both
    at the fp16 gate tolerance against the float64 head over the same fp16 inputs."""
    n_q = n_kv = 4
    d = 64
    L = past + c
    kp, vp, tables, qsl, q, bt = _ragged_case([L], [c], n_q, n_kv, d, torch.float16, L + c,
                                              poison=False)
    g = seeded(L)
    q = (8 * torch.randn(c, n_q, d, generator=g)).half()
    kp = (8 * kp.float()).half()
    sink_dir = q.float().mean(dim=0)  # (n_q, d): the queries' common direction per head
    for pos in range(4):
        blk, off = tables[0][pos // BLOCK_SIZE], pos % BLOCK_SIZE
        kp[:, blk, off] = (0.6 * sink_dir / sink_dir.norm(dim=-1, keepdim=True) * 64).half()
    got = _run_ragged(device, kp, vp, qsl, [L], bt, q, d**-0.5)
    for h in range(n_q):
        kh = op.gather_pool(kp.double(), tables[0], L)[h]
        vh = op.gather_pool(vp.double(), tables[0], L)[h]
        ref = oa.attention_f64(q[:, h], kh, vh, past, d**-0.5)
        torch.testing.assert_close(got[:, h].double(), ref, **FP16_TOL)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n_req", [2, 64])
def test_gqa8_workgroup_rows_take_query_vectors_in_passes(device, dtype, n_req) -> None:
    """Groups of 8 query heads per kv head (32 / 4) in workgroup rows: 64 decodes of at most
    4,096 tokens make one 16-wave workgroup per (request, kv head), 2 decodes are cut into parts
    of 8-wave workgroups, and both take their 8 query vectors in passes of 4. Against the oracle,
    slack poisoned."""
    n_q, n_kv, d = 32, 4, 64
    g = seeded(300 + n_req)
    lens = [int(x) for x in torch.randint(300, 4097, (n_req,), generator=g)]
    kp, vp, tables, qsl, q, bt = _ragged_case(lens, [1] * n_req, n_q, n_kv, d, dtype,
                                              90 + n_req)
    plan_host, _ = kernels.make_plan_host(qsl, np.asarray(lens, np.int32), n_q, n_kv, d,
                                          BLOCK_SIZE, bt.shape[1], dtype)
    assert int(plan_host[19]) == (16 if n_req == 64 else 8)  # workgroup rows / context parts
    assert int(plan_host[14]) == 8  # query vectors per row item
    got = _run_ragged(device, kp, vp, qsl, lens, bt, q, d**-0.5)
    expected = oa.ragged_reference(q, kp, vp, qsl.tolist(), lens, tables, d**-0.5)
    if dtype == torch.float32:
        tol = FP32_TOL
    elif dtype == torch.float16:
        tol = FP16_TOL
    else:  # bf16 keeps 8 bits of mantissa where fp16 keeps 11
        tol = {k_: v_ * 8 for k_, v_ in FP16_TOL.items()}
    torch.testing.assert_close(got.float(), expected, **tol)
