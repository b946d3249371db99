"""edgerag_paged_attention_noalloc: the attention entry point that allocates nothing.

It keeps the split partials in the library's static per-GPU scratch instead of a caller's
workspace; everything else is edgerag_paged_attention. The GPU tests call both entry points
through the C ABI on the same plan and inputs and require the same bits, on two calls in a row
(the second smaller than the first, so leftovers of the first sit in the scratch), and pin the
results against the CPU oracle at the north_star fp16 tolerance (atol 2e-3 / rtol 1e-2).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from edgerag_amd import _lib, kernels
from oracle import attention as oa
from tests.conftest import seeded

BS = 16
FP16_TOL = dict(rtol=1e-2, atol=2e-3)


def _batch(lens, q_lens, n_q, n_kv, seed, device):
    """Seeded ragged fp16 batch, pools drawn on the device; tables from one permutation."""
    g = seeded(seed)
    nbs = [math.ceil(L / BS) for L in lens]
    NB = sum(nbs) + 8
    perm = torch.randperm(NB, generator=g).numpy().astype(np.int32)
    bt = np.full((len(lens), max(nbs)), -1, np.int32)
    tables, at = [], 0
    for r, nb in enumerate(nbs):
        bt[r, :nb] = perm[at : at + nb]
        tables.append(perm[at : at + nb].tolist())
        at += nb
    gd = torch.Generator(device=device).manual_seed(seed)
    kp = torch.randn((n_kv, NB, BS, 64), generator=gd, device=device, dtype=torch.float16)
    vp = torch.randn((n_kv, NB, BS, 64), generator=gd, device=device, dtype=torch.float16)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    q = torch.randn((int(qsl[-1]), n_q, 64), generator=gd, device=device, dtype=torch.float16)
    return kp, vp, q, qsl, np.asarray(lens, np.int32), bt, tables


def _both(kp, vp, q, qsl, lens, bt, n_q, n_kv, device):
    """The same plan through edgerag_paged_attention (workspace) and the no-alloc entry. Decode
    rows are planned as KV splits, so they too leave partials in the scratch."""
    plan_ws, _ = kernels.plan_attention(qsl, lens, bt, n_q, n_kv, 64, BS, torch.float16, device,
                                        split_rows=True)
    plan_na, _ = kernels.plan_attention(qsl, lens, bt, n_q, n_kv, 64, BS, torch.float16, device,
                                        workspace=False, split_rows=True)
    assert plan_na.workspace is None and plan_na.workspace_bytes == plan_ws.workspace_bytes
    assert 0 < plan_na.workspace_bytes <= _lib.ATTN_SCRATCH_BYTES
    ref = kernels.paged_attention(q, kp, vp, plan_ws, 0.125, overlap=False)
    out = torch.full_like(q, float("nan"))
    got = kernels.paged_attention_noalloc(q, kp, vp, plan_na, 0.125, out=out)
    torch.cuda.synchronize()
    return ref, got, plan_na


@pytest.mark.gpu
def test_noalloc_equals_the_workspace_entry_on_two_calls(device) -> None:
    """Call 1: the config-3 prefill slices alone (3 slices of 512 at offsets 0 / 3584 / 6656,
    32/32 heads): MFMA tiles split over the keys, 21.6 MB of partials. Call 2: a smaller decode
    batch with split contexts. Each equals edgerag_paged_attention bit for bit."""
    lens1 = [512, 3584 + 512, 6656 + 512]
    q1 = [512, 512, 512]
    print("noalloc call 1: 3 prefill slices, 1536 tokens", flush=True)
    kp, vp, q, qsl, lens, bt, tables = _batch(lens1, q1, 32, 32, 303, device)
    ref1, got1, plan1 = _both(kp, vp, q, qsl, lens, bt, 32, 32, device)
    assert plan1.workspace_bytes > 16 << 20
    assert torch.equal(got1, ref1)
    del kp, vp

    lens2 = [300, 2900, 5100, 1000, 4400, 777]
    print("noalloc call 2: 6 decodes, 8/4 heads", flush=True)
    kp, vp, q, qsl, lens, bt, tables = _batch(lens2, [1] * 6, 8, 4, 304, device)
    ref2, got2, plan2 = _both(kp, vp, q, qsl, lens, bt, 8, 4, device)
    assert 0 < plan2.workspace_bytes < plan1.workspace_bytes
    assert torch.equal(got2, ref2)
    expected = oa.ragged_reference(q.cpu(), kp.cpu(), vp.cpu(), qsl.tolist(), lens2, tables, 0.125)
    torch.testing.assert_close(got2.float().cpu(), expected, **FP16_TOL)


@pytest.mark.gpu
def test_noalloc_parts_on_two_streams(device) -> None:
    """Prefill tiles on the current stream beside decode rows on a side stream, then the merge,
    all through the no-alloc entry (one step split in parts shares the scratch without racing:
    its parts write disjoint partials)."""
    lens_, q_ = [600, 2000 + 256, 3000, 4500, 800], [600, 256, 1, 1, 1]
    print("noalloc parts: 2 prefill slices + 3 decodes on two streams", flush=True)
    kp, vp, q, qsl, lens, bt, tables = _batch(lens_, q_, 8, 8, 305, device)
    ref, _, plan = _both(kp, vp, q, qsl, lens, bt, 8, 8, device)
    assert 0 < int(plan.plan_host[13]) < int(plan.plan_host[2])  # rows and tiles
    out = torch.full_like(q, float("nan"))
    main = torch.cuda.current_stream(device)
    side = torch.cuda.Stream(device)
    side.wait_stream(main)
    kernels.paged_attention_noalloc(q, kp, vp, plan, 0.125, out,
                                    parts=_lib.ATTN_TILES | _lib.ATTN_TILES_SHARED)
    with torch.cuda.stream(side):
        kernels.paged_attention_noalloc(q, kp, vp, plan, 0.125, out, parts=_lib.ATTN_ROWS)
    main.wait_stream(side)
    kernels.paged_attention_noalloc(q, kp, vp, plan, 0.125, out, parts=_lib.ATTN_COMBINE)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_noalloc_refuses_plans_beyond_the_scratch() -> None:
    """A plan whose partials exceed the static scratch is refused on the host, before any HIP
    call (no device pointer is even looked at), with EDGERAG_EWORKSPACE and a message."""
    n_q = n_kv = 128
    lens = np.full(128, 7472, np.int32)  # 128 decodes x 128 heads x 8 splits: 34.6 MB
    qsl = np.arange(129, dtype=np.int32)
    plan, ws = kernels.make_plan_host(qsl, lens, n_q, n_kv, 64, BS, 467, torch.float16,
                                      split_rows=True)
    assert ws > _lib.ATTN_SCRATCH_BYTES
    lib = _lib.load()
    rc = lib.edgerag_paged_attention_noalloc(
        plan.ctypes.data, None, plan.size, None, 0, 0, None, None, 1, None, 0, None, None, 128, 128,
        n_q, n_kv, 64, BS, 16384, 0.125, None, 0, 0, _lib.ATTN_ALL, None)
    assert rc == _lib.EDGERAG_EWORKSPACE
    msg = lib.edgerag_last_error().decode()
    assert "static scratch holds" in msg and str(_lib.ATTN_SCRATCH_BYTES) in msg
