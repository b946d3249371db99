"""Preemption (edgerag/cache/preemption.py): swap-out/in round trips of the head-major pools,
allocator accounting, victim order and the policies. CPU pools; the device path is in
tests/test_gpu_kv.py."""

from __future__ import annotations

import pytest
import torch

from edgerag_amd.cache.allocator import BlockAllocator, OutOfBlocksError
from edgerag_amd.cache.preemption import PreemptionPolicy, Preemptor
from tests.conftest import seeded


def _pools(layers=3, heads=4, blocks=32, bs=16, d=8):
    g = seeded(layers * 100 + heads)
    kp = [torch.randn(heads, blocks, bs, d, generator=g).half() for _ in range(layers)]
    vp = [torch.randn(heads, blocks, bs, d, generator=g).half() for _ in range(layers)]
    return kp, vp


def test_swap_round_trip_restores_every_layer_at_new_blocks() -> None:
    alloc = BlockAllocator(32, 16)
    kp, vp = _pools()
    blocks = alloc.allocate(5)
    saved_k = [p[:, blocks].clone() for p in kp]
    saved_v = [p[:, blocks].clone() for p in vp]
    pre = Preemptor(alloc, pin_memory=False)
    rec = pre.swap_out("a", blocks, 70, kp, vp)
    assert rec.num_blocks == 5 and alloc.num_free == 32
    assert rec.nbytes == 2 * 3 * 4 * 5 * 16 * 8 * 2
    other = alloc.allocate(5)  # another sequence takes (and overwrites) the freed blocks
    for p in kp + vp:
        p[:, other] = 0
    new_blocks, n = pre.swap_in("a", kp, vp)
    assert n == 70 and len(new_blocks) == 5 and not set(new_blocks) & set(other)
    for layer in range(3):
        assert torch.equal(kp[layer][:, new_blocks], saved_k[layer])
        assert torch.equal(vp[layer][:, new_blocks], saved_v[layer])
    assert pre.swapped == {} and pre.stats.swaps_out == 1 and pre.stats.swaps_in == 1
    alloc.check_invariants()


def test_swap_in_without_room_changes_nothing() -> None:
    alloc = BlockAllocator(8, 16)
    kp, vp = _pools(blocks=8)
    pre = Preemptor(alloc, pin_memory=False)
    pre.swap_out("a", alloc.allocate(6), 90, kp, vp)
    hog = alloc.allocate(4)
    with pytest.raises(OutOfBlocksError):
        pre.swap_in("a", kp, vp)
    assert "a" in pre.swapped and alloc.num_free == 4
    alloc.free(hog)
    blocks, _ = pre.swap_in("a", kp, vp)
    assert len(blocks) == 6
    with pytest.raises(KeyError):
        pre.swap_in("a", kp, vp)


@pytest.mark.parametrize("policy", list(PreemptionPolicy))
def test_policies_return_the_freed_blocks(policy) -> None:
    alloc = BlockAllocator(16, 16)
    kp, vp = _pools(blocks=16)
    pre = Preemptor(alloc, policy=policy, pin_memory=False)
    blocks = alloc.allocate(3)
    assert pre.preempt("r", blocks, 40, kp, vp) == 3
    assert alloc.num_free == 16 and pre.stats.preemptions == 1
    d = pre.to_dict()
    assert d["policy"] == policy.value and d["blocks_reclaimed"] == 3
    assert d["num_swapped"] == (1 if policy is PreemptionPolicy.SWAP else 0)
    assert d["recomputes"] == (policy is PreemptionPolicy.RECOMPUTE)
    assert d["rejects"] == (policy is PreemptionPolicy.REJECT)
    if policy is PreemptionPolicy.SWAP:
        with pytest.raises(ValueError):
            pre.preempt("s", alloc.allocate(1), 5)


def test_victims_newest_first_until_covered() -> None:
    cands = [("old", 4), ("mid", 2), ("new", 3)]
    assert Preemptor.select_victims(cands, 0) == []
    assert Preemptor.select_victims(cands, 3) == ["new"]
    assert Preemptor.select_victims(cands, 4) == ["new", "mid"]
    assert Preemptor.select_victims(cands, 100) == ["new", "mid", "old"]
