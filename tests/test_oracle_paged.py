"""Pins of the paged-pool oracle (oracle/paged.py, oracle/c): CPU only.

The torch restatement of PagedKVCache._write / _gather_pool (edgerag/cache/paged.py:186-238)
is checked against (1) the closed form slot = table[p // bs] * bs + p % bs, (2) a per-token
brute-force loop over BlockTable.locate (block_table.py:48-60), and (3) an independent C
restatement that moves raw bytes. A planted off-by-one in the slot arithmetic must fail (1).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import c_oracle
from oracle import paged as op
from tests.conftest import seeded


@pytest.mark.parametrize(
    "tokens,bs,expected", [(0, 16, 0), (1, 16, 1), (15, 16, 1), (16, 16, 1), (17, 16, 2),
                           (32, 16, 2), (33, 16, 3), (7472, 16, 467), (5, 1, 5)]
)
def test_blocks_needed_is_exact_ceil(tokens, bs, expected) -> None:
    """allocator.py:244-254 and test_paged.py:185-194: no spare block at exact multiples."""
    assert op.blocks_needed(tokens, bs) == expected


@given(
    n_blocks=st.integers(1, 12),
    bs=st.sampled_from([1, 2, 8, 16, 32]),
    data=st.data(),
)
@settings(max_examples=60, deadline=None)
def test_slot_mapping_closed_form_equals_locate_loop(n_blocks, bs, data) -> None:
    table = data.draw(st.permutations(list(range(n_blocks + 5))))[:n_blocks]
    cap = n_blocks * bs
    start = data.draw(st.integers(0, cap - 1))
    n = data.draw(st.integers(1, cap - start))
    got = op.slot_mapping(table, start, n, bs).tolist()
    brute = [table[p // bs] * bs + p % bs for p in range(start, start + n)]
    assert got == brute


def test_planted_off_by_one_in_slot_arithmetic_is_caught() -> None:
    """A mistake a kernel could make ((p + 1) // bs) must disagree with the oracle."""
    table, bs = [7, 2, 5], 16
    good = op.slot_mapping(table, 10, 30, bs).tolist()
    planted = [table[min((p + 1) // bs, 2)] * bs + p % bs for p in range(10, 40)]
    assert good != planted


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("bs,start,n", [(16, 0, 1), (16, 15, 2), (8, 3, 37), (32, 40, 100)])
def test_write_slots_matches_bruteforce_and_c(dtype, bs, start, n) -> None:
    g = seeded(bs * 1000 + start * 7 + n)
    H, D = 3, 64
    nb = op.blocks_needed(start + n, bs)
    NB = nb + 4
    table = torch.randperm(NB, generator=g)[:nb].tolist()
    pool = torch.randn(H, NB, bs, D, generator=g).to(dtype)
    src = torch.randn(1, H, n, D, generator=g).to(dtype)
    a, b = pool.clone(), pool.clone()
    op.write_slots(a, src, table, start)
    op.write_slots_bruteforce(b, src, table, start)
    assert torch.equal(a, b)
    c = pool.clone().numpy()
    c_oracle.slot_scatter(c, src[0].numpy(), table, start)
    assert np.array_equal(c, a.numpy())
    # untouched blocks really are untouched
    untouched = sorted(set(range(NB)) - set(table))
    assert torch.equal(a[:, untouched], pool[:, untouched])


@pytest.mark.parametrize("seq_len", [1, 15, 16, 17, 33, 64, 100])
def test_gather_returns_exactly_seq_len_and_matches_c(seq_len) -> None:
    """The P-01 slice (paged.py:237-238): the final block's slack is never returned."""
    g = seeded(seq_len)
    bs, H, D = 16, 2, 8
    nb = op.blocks_needed(seq_len, bs)
    pool = torch.randn(H, nb + 2, bs, D, generator=g)
    table = torch.randperm(nb + 2, generator=g)[:nb].tolist()
    out = op.gather_pool(pool, table, seq_len)
    assert out.shape == (H, seq_len, D)
    assert np.array_equal(c_oracle.gather(pool.numpy(), table, seq_len), out.numpy())
    for p in (0, seq_len - 1):
        assert torch.equal(out[:, p], pool[:, table[p // bs], p % bs])
