"""KV append / gather / block copy on the GPU, bit-exact against the oracle.

Pins (reference): ``PagedKVCache._write`` (edgerag/cache/paged.py:186-206), ``gather``
(:208-238), the CoW content copy (:151-182) and the CoW tensor tests of tests/test_cow.py.
"""

from __future__ import annotations

import pytest
import torch

from edgerag_amd import kernels
from edgerag_amd.cache.allocator import BlockAllocator
from edgerag_amd.cache.paged import PagedKVCache
from edgerag_amd.core.spec import ModelSpec
from oracle import paged as op
from tests.conftest import seeded

pytestmark = pytest.mark.gpu

CFG1_LENS = [37, 128, 300, 511]
CFG1_SPLIT = [3, 8, 19, 32]


def cfg1_tables(seed: int = 1) -> list[list[int]]:
    perm = torch.randperm(64, generator=seeded(seed)).tolist()
    out, at = [], 0
    for n in CFG1_SPLIT:
        out.append(perm[at : at + n])
        at += n
    return out


def test_cfg1_append_of_four_new_tokens_is_bit_exact(device) -> None:
    """cfg1: four sequences append one token each; whole pools compared with torch.equal."""
    g = seeded(0)
    H, NB, BS, D = 3, 64, 16, 64
    key_pool = torch.randn(H, NB, BS, D, generator=g)
    value_pool = torch.randn(H, NB, BS, D, generator=g)
    tables = cfg1_tables()
    new_k = torch.randn(4, H, D, generator=g)
    new_v = torch.randn(4, H, D, generator=g)

    exp_k, exp_v = key_pool.clone(), value_pool.clone()
    slots = []
    for r, L in enumerate(CFG1_LENS):
        op.write_slots(exp_k, new_k[r][None, :, None], tables[r], L - 1)
        op.write_slots(exp_v, new_v[r][None, :, None], tables[r], L - 1)
        slots.append(int(op.slot_mapping(tables[r], L - 1, 1, BS)[0]))

    dk, dv = key_pool.to(device), value_pool.to(device)
    kernels.kv_append(
        new_k.to(device), new_v.to(device), torch.tensor(slots, dtype=torch.int32, device=device),
        dk, dv,
    )
    assert torch.equal(dk.cpu(), exp_k)
    assert torch.equal(dv.cpu(), exp_v)


@pytest.mark.parametrize("block_size", [8, 16, 32])
@pytest.mark.parametrize("start,n_new", [(0, 1), (15, 2), (16, 16), (20, 37), (0, 512)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
def test_chunk_append_matches_oracle(device, block_size, start, n_new, dtype) -> None:
    g = seeded(start * 131 + n_new)
    H, D = 4, 64
    n_blocks_needed = op.blocks_needed(start + n_new, block_size)
    NB = n_blocks_needed + 5
    table = torch.randperm(NB, generator=g)[:n_blocks_needed].tolist()
    pool = torch.randn(H, NB, block_size, D, generator=g).to(dtype)
    src = torch.randn(1, H, n_new, D, generator=g).to(dtype)
    expected = pool.clone()
    op.write_slots(expected, src, table, start)
    brute = pool.clone()
    op.write_slots_bruteforce(brute, src, table, start)
    assert torch.equal(expected, brute)

    dpool = pool.to(device)
    slots = op.slot_mapping(table, start, n_new, block_size).to(torch.int32).to(device)
    kernels.kv_append(src[0].transpose(0, 1).to(device), None, slots, dpool, None)
    assert torch.equal(dpool.cpu(), expected)


def test_fp32_source_into_fp16_pool_rounds_like_tensor_to(device) -> None:
    """``.to(pool.dtype)`` (paged.py:206): round-to-nearest-even, bit for bit."""
    g = seeded(5)
    H, NB, BS, D = 2, 8, 16, 64
    pool = torch.zeros(H, NB, BS, D, dtype=torch.float16)
    src = (torch.randn(1, H, 19, D, generator=g) * 1000).float()
    table = [5, 1]
    expected = pool.clone()
    op.write_slots(expected, src, table, 3)
    dpool = pool.to(device)
    slots = op.slot_mapping(table, 3, 19, BS).to(torch.int32).to(device)
    kernels.kv_append(src[0].transpose(0, 1).to(device), None, slots, dpool, None)
    assert torch.equal(dpool.cpu(), expected)


def test_negative_and_out_of_pool_slots_are_skipped(device) -> None:
    H, NB, BS, D = 2, 4, 16, 64
    pool = torch.zeros(H, NB, BS, D, dtype=torch.float16, device=device)
    src = torch.ones(3, H, D, dtype=torch.float16, device=device)
    slots = torch.tensor([-1, 5, NB * BS + 7], dtype=torch.int32, device=device)
    kernels.kv_append(src, None, slots, pool, None)
    flat = pool.view(H, NB * BS, D).cpu()
    assert flat[:, 5].eq(1).all()
    assert flat.sum().item() == H * D  # only slot 5 was written


@pytest.mark.parametrize("seq_len", [1, 2, 15, 16, 17, 31, 32, 33, 47, 48, 49, 63, 64, 65, 100, 129])
def test_gather_returns_exactly_seq_len_tokens(device, seq_len) -> None:
    g = seeded(seq_len)
    H, BS, D = 3, 16, 64
    nb = op.blocks_needed(seq_len, BS)
    NB = nb + 3
    pool = torch.randn(H, NB, BS, D, generator=g).half()
    table = torch.randperm(NB, generator=g)[:nb].tolist()
    expected = op.gather_pool(pool, table, seq_len)
    got = kernels.kv_gather(pool.to(device), torch.tensor(table, device=device), seq_len)
    assert got.shape == (H, seq_len, D)
    assert torch.equal(got.cpu(), expected)


def test_copy_blocks_moves_every_head(device) -> None:
    g = seeded(9)
    pool = torch.randn(4, 10, 16, 64, generator=g).half()
    expected = pool.clone()
    expected[:, [7, 2]] = pool[:, [1, 3]]
    dpool = pool.to(device)
    kernels.kv_copy_blocks(
        dpool, torch.tensor([1, 3], device=device), torch.tensor([7, 2], device=device)
    )
    assert torch.equal(dpool.cpu(), expected)


# --- the cache object ------------------------------------------------------------------------

BLOCK = 8


def tiny_spec(n_layers: int = 2) -> ModelSpec:
    return ModelSpec(
        model_id="tiny", model_type="test", n_layers=n_layers, hidden_size=32, n_q_heads=4,
        n_kv_heads=2, head_dim=8, vocab_size=100, max_position_embeddings=128,
        rope_theta=10000.0, pad_token_id=0, intermediate_size=64,
    )


def make_cache(allocator, device, spec=None) -> PagedKVCache:
    return PagedKVCache(spec or tiny_spec(), allocator, device, torch.float32)


def fill(cache: PagedKVCache, n_tokens: int, value: float) -> None:
    spec = cache.spec
    kv = torch.full((1, spec.n_kv_heads, n_tokens, spec.head_dim), value, device=cache.device)
    for layer in range(spec.n_layers):
        cache.update(kv, kv, layer)


def test_update_returns_the_appended_history(device) -> None:
    allocator = BlockAllocator(16, BLOCK)
    cache = make_cache(allocator, device)
    g = seeded(3)
    chunks = [torch.randn(1, 2, n, 8, generator=g) for n in (5, 1, 11, 1)]
    for c in chunks:
        for layer in range(2):
            keys, values = cache.update(c.to(device), (c * 2).to(device), layer)
    history = torch.cat(chunks, dim=2)
    assert cache.seq_len == history.shape[2]
    assert torch.equal(keys.cpu(), history)
    assert torch.equal(values.cpu(), history * 2)
    assert len(cache.table.blocks) == op.blocks_needed(cache.seq_len, BLOCK)


def test_sibling_writes_do_not_corrupt_each_other(device) -> None:
    """tests/test_cow.py:62-88 restated on device tensors."""
    allocator = BlockAllocator(16, BLOCK)
    parent = make_cache(allocator, device)
    fill(parent, 10, 1.0)
    child = parent.fork()
    child_before = child.gather(0)[0].clone()
    fill(child, 3, 7.0)
    assert torch.equal(parent.gather(0)[0], child_before[:, :10])
    fill(parent, 3, -5.0)
    child_after = child.gather(0)[0]
    assert not (child_after == -5.0).any()
    assert (child_after[:, 10:13] == 7.0).all()
    allocator.check_invariants()


def test_copy_on_write_copies_contents_once_for_every_layer(device) -> None:
    """tests/test_cow.py:91-115: content copy, and one split per forward, not per layer."""
    allocator = BlockAllocator(16, BLOCK)
    parent = make_cache(allocator, device, tiny_spec(n_layers=6))
    fill(parent, 10, 3.0)
    child = parent.fork()
    fill(child, 2, 9.0)
    assert allocator.counters.private_copies == 1
    for layer in range(6):
        keys, _ = child.gather(layer)
        assert (keys[0, :, :10] == 3.0).all()
        assert (keys[0, :, 10:12] == 9.0).all()


def test_swap_out_in_on_device_pools(device) -> None:
    """Swap-out gathers the victim's blocks of every layer with edgerag_kv_gather into a device
    staging buffer and copies it to pinned host memory on the stream, before the blocks are
    freed: a kernel that reuses them right after (on the same stream) cannot change the swapped
    copy. Swap-in scatters it back with edgerag_kv_append: every layer bit for bit at the newly
    allocated blocks."""
    from edgerag_amd.cache.allocator import BlockAllocator
    from edgerag_amd.cache.preemption import Preemptor

    g = torch.Generator(device=device).manual_seed(3)
    layers, heads, nb, bs, d = 4, 8, 64, 16, 64
    kp = [torch.randn(heads, nb, bs, d, generator=g, device=device).half() for _ in range(layers)]
    vp = [torch.randn(heads, nb, bs, d, generator=g, device=device).half() for _ in range(layers)]
    alloc = BlockAllocator(nb, bs)
    blocks = alloc.allocate(9)
    saved_k = [p[:, blocks].clone() for p in kp]
    saved_v = [p[:, blocks].clone() for p in vp]
    pre = Preemptor(alloc)
    rec = pre.swap_out("v", blocks, 130, kp, vp)
    other = alloc.allocate(nb)  # every block, the victim's included, is reused at once
    for p in kp + vp:
        p[:, other] = 0
    for layer in range(layers):  # reading the record waits for the copy
        k, v = rec.layer(layer)
        assert k.is_pinned() and torch.equal(k, saved_k[layer].cpu())
        assert torch.equal(v, saved_v[layer].cpu())
    alloc.free(other)
    new_blocks, n = pre.swap_in("v", kp, vp)
    assert n == 130 and len(new_blocks) == 9
    for layer in range(layers):
        assert torch.equal(kp[layer][:, new_blocks], saved_k[layer])
        assert torch.equal(vp[layer][:, new_blocks], saved_v[layer])
    alloc.check_invariants()


def test_swap_in_without_room_keeps_the_record(device) -> None:
    from edgerag_amd.cache.allocator import BlockAllocator, OutOfBlocksError
    from edgerag_amd.cache.preemption import Preemptor

    kp = [torch.randn(2, 8, 16, 64, device=device).half()]
    vp = [torch.randn(2, 8, 16, 64, device=device).half()]
    alloc = BlockAllocator(8, 16)
    pre = Preemptor(alloc)
    pre.swap_out("a", alloc.allocate(6), 90, kp, vp)
    hog = alloc.allocate(4)
    with pytest.raises(OutOfBlocksError):
        pre.swap_in("a", kp, vp)
    assert "a" in pre.swapped and alloc.num_free == 4
    alloc.free(hog)
    blocks, n = pre.swap_in("a", kp, vp)
    assert len(blocks) == 6 and n == 90
    with pytest.raises(KeyError):
        pre.swap_in("a", kp, vp)


def test_reference_executor_call_sequence(device) -> None:
    """The reference executor's order (``edgerag/serve/executor.py:124-128``, ``:151-153``):
    ``table.ensure_capacity(seq_len + n)`` first, then ``update(k, v, layer)`` for every layer.
    The pre-grown table takes no further block, and each layer's history is exact."""
    allocator = BlockAllocator(16, BLOCK)
    cache = make_cache(allocator, device)
    g = seeded(4)
    chunks = [torch.randn(1, 2, n, 8, generator=g) for n in (21, 1, 16, 1, 3)]
    for c in chunks:
        cache.table.ensure_capacity(cache.seq_len + c.shape[2])
        used = allocator.num_used
        for layer in range(2):
            keys, values = cache.update(c.to(device), (c * 3).to(device), layer)
        assert allocator.num_used == used
    history = torch.cat(chunks, dim=2)
    assert cache.seq_len == history.shape[2]
    assert torch.equal(keys.cpu(), history) and torch.equal(values.cpu(), history * 3)
    assert len(cache.table.blocks) == op.blocks_needed(cache.seq_len, BLOCK)
    allocator.check_invariants()
