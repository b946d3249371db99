"""Preemption policies and victim order (host only). The block movement of a swap runs the HIP
kernels and is tested on device pools in tests/test_gpu_kv.py."""

from __future__ import annotations

import types

import pytest

from edgerag_amd.cache.allocator import BlockAllocator
from edgerag_amd.cache.block_table import BlockTable
from edgerag_amd.cache.preemption import PreemptionPolicy, Preemptor


def _request(alloc, n_tokens):
    table = BlockTable(alloc)
    table.append(n_tokens)
    cache = types.SimpleNamespace(table=table, key_pool=None, value_pool=None)
    return types.SimpleNamespace(request_id="r", cache=cache, swap=None)


@pytest.mark.parametrize("policy", [PreemptionPolicy.RECOMPUTE, PreemptionPolicy.REJECT])
def test_policies_without_a_swap(policy) -> None:
    alloc = BlockAllocator(16, 16)
    pre = Preemptor(alloc, policy=policy)
    req = _request(alloc, 40)
    assert pre.evict(req) == policy.value
    assert req.cache.table.num_blocks == 3  # the scheduler drops the cache
    snap = pre.snapshot()
    assert snap["policy"] == policy.value and snap["events"]["evicted"] == 1


def test_swap_refuses_host_pools() -> None:
    """There is no CPU path: swapping host tensors is an error, not a silent torch copy."""
    import torch

    alloc = BlockAllocator(8, 16)
    pools = [torch.zeros(2, 8, 16, 8, dtype=torch.float16)]
    with pytest.raises(ValueError, match="MI355X"):
        Preemptor(alloc).swap_out("r", alloc.allocate(2), 20, pools, pools)


def test_victims_newest_first_until_covered() -> None:
    cands = [("old", 4), ("mid", 2), ("new", 3)]
    assert Preemptor.select_victims(cands, 0) == []
    assert Preemptor.select_victims(cands, 3) == ["new"]
    assert Preemptor.select_victims(cands, 4) == ["new", "mid"]
    assert Preemptor.select_victims(cands, 100) == ["new", "mid", "old"]
