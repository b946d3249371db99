"""Pins of the attention oracle (oracle/attention.py): CPU only.

paged_attention_reference (edgerag/cache/fused.py:89-167) and ragged_reference (executor loop
over build_causal_mask + sdpa_attention, edgerag/core/layers.py:137-167, :227-254) are checked
against a float64 textbook softmax (attention_f64), against torch SDPA special cases, and with
the reference's own test cases (tests/test_fused_attention.py). Each planted mistake a kernel
could plausibly make -- tiled instead of interleaved GQA heads, an off-by-one causal mask, a
missing scale, an attended slack slot -- must fail one of these checks.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as oa
from oracle import paged as op
from tests.conftest import seeded

BS = 16


def _pool(h, nb, d, g):
    return torch.randn(h, nb, BS, d, generator=g), torch.randn(h, nb, BS, d, generator=g)


def _per_head_f64(q, kp, vp, table, L, past, scale, n_rep):
    """float64 attention per query head, kv head = q_head // n_rep."""
    k = op.gather_pool(kp, table, L)
    v = op.gather_pool(vp, table, L)
    outs = [oa.attention_f64(q[:, hq], k[hq // n_rep], v[hq // n_rep], past, scale)
            for hq in range(q.shape[1])]
    return torch.stack(outs, dim=1)  # (c, H_q, d)


@pytest.mark.parametrize(
    "seq_len", [1, 2, 15, 16, 17, 31, 32, 33, 47, 48, 49, 63, 64, 65, 100, 127, 128, 129]
)
def test_blockwise_spec_matches_gather_sdpa_and_f64(seq_len) -> None:
    """test_fused_attention.py:71-91, plus the float64 closed form."""
    g = seeded(seq_len)
    nb = math.ceil(seq_len / BS)
    kp, vp = _pool(4, nb + 3, 8, g)
    ids = torch.randperm(nb + 3, generator=g)[:nb]
    q = torch.randn(1, 4, 1, 8, generator=g)
    spec = oa.paged_attention_reference(q, kp, vp, ids, seq_len, 8**-0.5)
    torch.testing.assert_close(spec, oa.sdpa_over_gather(q, kp, vp, ids, seq_len, 8**-0.5, 1),
                               rtol=1e-5, atol=1e-5)
    f64 = _per_head_f64(q[0].transpose(0, 1), kp, vp, ids.tolist(), seq_len, seq_len - 1,
                        8**-0.5, 1)
    torch.testing.assert_close(spec[0].double(), f64, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("n_rep", [1, 2, 3, 4])
def test_gqa_interleaved_heads_and_planted_tiling_is_caught(n_rep) -> None:
    """layers.py:117-134 (P-08): kv = q_head // n_rep; torch.repeat's tiling must differ."""
    g = seeded(n_rep)
    kp, vp = _pool(3, 5, 8, g)
    ids = torch.tensor([0, 1, 2])
    q = torch.randn(1, 3 * n_rep, 1, 8, generator=g)
    spec = oa.paged_attention_reference(q, kp, vp, ids, 40, 8**-0.5, n_rep)
    f64 = _per_head_f64(q[0].transpose(0, 1), kp, vp, [0, 1, 2], 40, 39, 8**-0.5, n_rep)
    torch.testing.assert_close(spec[0].double(), f64, rtol=1e-5, atol=1e-6)
    if n_rep > 1:
        k = op.gather_pool(kp, [0, 1, 2], 40)
        v = op.gather_pool(vp, [0, 1, 2], 40)
        tiled = torch.stack([oa.attention_f64(q[0, hq], k[hq % 3], v[hq % 3], 39, 8**-0.5)[0]
                             for hq in range(3 * n_rep)])
        assert not torch.allclose(tiled, f64[0], atol=1e-3)


def test_poisoned_slack_and_extra_blocks_change_nothing() -> None:
    """test_fused_attention.py:94-131; a planted read of one slack slot must be visible."""
    g = seeded(17)
    kp, vp = _pool(2, 6, 8, g)
    q = torch.randn(1, 2, 1, 8, generator=g)
    clean = oa.paged_attention_reference(q, kp, vp, torch.tensor([0, 1]), 17, 8**-0.5)
    kp[:, 1, 1:] = 1e4
    vp[:, 1, 1:] = 1e4
    kp[:, 2:] = 1e4
    vp[:, 2:] = 1e4
    poisoned = oa.paged_attention_reference(q, kp, vp, torch.tensor([0, 1, 2, 3]), 17, 8**-0.5)
    torch.testing.assert_close(poisoned, clean, rtol=1e-6, atol=1e-6)
    # Reading one slot too many (seq_len 18) must move the output: give that slot a finite
    # score (zero key) and a huge value.
    kp[:, 1, 1] = 0.0
    planted = oa.paged_attention_reference(q, kp, vp, torch.tensor([0, 1]), 18, 8**-0.5)
    assert (planted - clean).abs().max() > 1.0


def test_overflow_empty_and_guards() -> None:
    """test_fused_attention.py:175-223."""
    g = seeded(33)
    kp, vp = _pool(2, 4, 8, g)
    q = torch.randn(1, 2, 1, 8, generator=g) * 200.0
    out = oa.paged_attention_reference(q, kp * 200.0, vp, torch.tensor([0, 1, 2]), 33, 8**-0.5)
    assert torch.isfinite(out).all()
    zero = oa.paged_attention_reference(q, kp, vp, torch.tensor([0]), 0, 8**-0.5)
    assert torch.count_nonzero(zero) == 0
    with pytest.raises(ValueError, match="decode path"):
        oa.paged_attention_reference(torch.randn(1, 2, 7, 8), kp, vp, torch.tensor([0]), 16, 1.0)
    with pytest.raises(ValueError, match="query heads"):
        oa.paged_attention_reference(torch.randn(1, 6, 1, 8), kp, vp, torch.tensor([0]), 16, 1.0)


def test_causal_mask_closed_form_and_planted_off_by_one() -> None:
    """layers.py:227-254: row i of a chunk at offset past sees keys k <= past + i."""
    mask = oa.build_causal_mask(4, 3, torch.float32)[0, 0]
    visible = (mask == 0).int()
    expected = torch.tensor([[1 if k <= 3 + i else 0 for k in range(7)] for i in range(4)])
    assert torch.equal(visible, expected)
    assert (mask[visible == 0] == torch.finfo(torch.float32).min).all()
    planted = torch.tensor([[1 if k < 3 + i else 0 for k in range(7)] for i in range(4)])
    assert not torch.equal(visible, planted)


def _ragged(lens, q_lens, n_q, n_kv, d, seed):
    g = seeded(seed)
    nbs = [math.ceil(L / BS) for L in lens]
    kp, vp = _pool(n_kv, sum(nbs) + 2, d, g)
    perm = torch.randperm(sum(nbs) + 2, generator=g).tolist()
    tables, at = [], 0
    for nb in nbs:
        tables.append(perm[at : at + nb])
        at += nb
    qsl = [0]
    for c in q_lens:
        qsl.append(qsl[-1] + c)
    q = torch.randn(qsl[-1], n_q, d, generator=g)
    return kp, vp, tables, qsl, q


def test_ragged_reference_equals_float64_per_request() -> None:
    lens, q_lens = [40, 101, 300, 17], [40, 37, 1, 5]
    kp, vp, tables, qsl, q = _ragged(lens, q_lens, 8, 4, 16, 3)
    out = oa.ragged_reference(q, kp, vp, qsl, lens, tables, 0.25)
    for r, (L, c) in enumerate(zip(lens, q_lens)):
        f64 = _per_head_f64(q[qsl[r] : qsl[r + 1]], kp, vp, tables[r], L, L - c, 0.25, 2)
        torch.testing.assert_close(out[qsl[r] : qsl[r + 1]].double(), f64, rtol=1e-5, atol=1e-6)


def test_single_chunk_without_prefix_is_causal_sdpa() -> None:
    kp, vp, tables, qsl, q = _ragged([77], [77], 4, 4, 16, 4)
    out = oa.ragged_reference(q, kp, vp, qsl, [77], tables, 0.25)
    k = op.gather_pool(kp, tables[0], 77)
    v = op.gather_pool(vp, tables[0], 77)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(0, 1), k, v, is_causal=True, scale=0.25
    ).transpose(0, 1)
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)
    # a planted missing scale is visible
    bad = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(0, 1), k, v, is_causal=True, scale=1.0
    ).transpose(0, 1)
    assert not torch.allclose(out, bad, atol=1e-3)


def test_chunked_equals_unchunked() -> None:
    """test_batched.py:80-119 / executor.py:51-54: the cached prefix is fully visible."""
    L = 150
    kp, vp, tables, _, q = _ragged([L], [L], 4, 2, 16, 5)
    whole = oa.ragged_reference(q, kp, vp, [0, L], [L], tables, 0.25)
    parts = [oa.ragged_reference(q[s:e], kp, vp, [0, e - s], [e], tables, 0.25)
             for s, e in ((0, 64), (64, 128), (128, 150))]
    torch.testing.assert_close(torch.cat(parts), whole, rtol=5e-5 * 3, atol=5e-5 * 3)


def test_eager_and_sdpa_restatements_agree() -> None:
    """layers.py:137-167 vs :192-224 (the reference's own 5e-3 band, test_equivalence.py:62)."""
    g = seeded(6)
    q = torch.randn(1, 4, 9, 16, generator=g)
    k = torch.randn(1, 2, 20, 16, generator=g)
    v = torch.randn(1, 2, 20, 16, generator=g)
    mask = oa.build_causal_mask(9, 11, torch.float32)
    torch.testing.assert_close(oa.sdpa_attention(q, k, v, mask, 0.25, 2),
                               oa.eager_attention(q, k, v, mask, 0.25, 2), rtol=5e-3, atol=5e-3)
