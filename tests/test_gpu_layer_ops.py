"""Fused layer ops (residual add + RMSNorm, RoPE + KV append, SiLU * up) against the decoder
oracle's restatement of ``edgerag/core/layers.py`` on the same inputs."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from edgerag_amd import kernels
from edgerag_amd.core.layers import RotaryTable
from oracle import model as om
from tests.conftest import seeded

pytestmark = pytest.mark.gpu


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Equal values, NaN matching NaN."""
    return bool(((a == b) | (a.isnan() & b.isnan())).all()) and a.shape == b.shape


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("width", [128, 2048, 8192, 1000])
def test_add_rmsnorm(device, dtype, width) -> None:
    g = seeded(width)
    x = torch.randn(13, width, generator=g).to(dtype)
    delta = torch.randn(13, width, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(width, generator=g)).to(dtype)
    h_ref = x + delta  # rounded to dtype, like the reference's residual add
    y_ref = om.rms_norm(h_ref, w, 1e-5)
    xd = x.to(device)
    y = kernels.rmsnorm(xd, w.to(device), 1e-5, delta=delta.to(device), h_out=xd)
    assert torch.equal(xd.cpu(), h_ref)
    tol = dict(rtol=0, atol=0) if dtype == torch.float32 else dict(rtol=2e-3, atol=2e-3)
    if dtype == torch.float32:
        torch.testing.assert_close(y.cpu(), y_ref, rtol=1e-5, atol=1e-5)
    else:
        torch.testing.assert_close(y.cpu().float(), y_ref.float(), **tol)
    y2 = kernels.rmsnorm(x.to(device), w.to(device), 1e-5)
    torch.testing.assert_close(y2.cpu().float(), om.rms_norm(x, w, 1e-5).float(),
                               rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("width", [64, 2048, 8192])
def test_embed_rmsnorm_equals_lookup_then_rmsnorm(device, dtype, width) -> None:
    """The embedding lookup fused into the first RMSNorm: bit for bit the rows of index_select
    (nn.Embedding, edgerag/core/model.py:109) and the RMSNorm of the same launch shape; ids
    outside the table give rows of NaN; widths that are not whole 16-byte chunks are refused."""
    g = seeded(width + 3)
    vocab = 500
    table = torch.randn(vocab, width, generator=g).to(dtype).to(device)
    w = (1 + 0.1 * torch.randn(width, generator=g)).to(dtype).to(device)
    ids = torch.tensor([3, 499, 0, 17, 3, 250, 1, 498], dtype=torch.int32)
    h, y, none = kernels.embed_rmsnorm(ids.to(device), table, w, 1e-5)
    assert none is None
    h_ref = table.index_select(0, ids.to(device))
    assert torch.equal(h, h_ref)
    assert torch.equal(y, kernels.rmsnorm(h_ref, w, 1e-5))
    # With the rotary rows gathered in the same launch: what rope_rows writes, positions outside
    # the table included (NaN rows); the embedding outputs unchanged.
    cos = torch.randn(300, 64, generator=g).to(dtype).to(device)
    sin = torch.randn(300, 64, generator=g).to(dtype).to(device)
    pos = torch.tensor([0, 299, 5, 300, -1, 17, 17, 128], dtype=torch.int32).to(device)
    h3, y3, (c3, s3) = kernels.embed_rmsnorm(ids.to(device), table, w, 1e-5, rope=(pos, cos, sin))
    c_ref, s_ref = kernels.rope_rows(pos, cos, sin)
    assert torch.equal(h3, h) and torch.equal(y3, y)
    assert _same(c3, c_ref) and _same(s3, s_ref) and c3[[3, 4]].isnan().all()
    tol = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 1.6e-2}[dtype]
    torch.testing.assert_close(y.cpu().float(), om.rms_norm(h_ref.cpu(), w.cpu(), 1e-5).float(),
                               rtol=tol, atol=tol)
    bad = torch.tensor([5, -1, vocab, 7], dtype=torch.int32)
    h2, y2, _ = kernels.embed_rmsnorm(bad.to(device), table, w, 1e-5)
    assert h2[[1, 2]].isnan().all() and y2[[1, 2]].isnan().all()
    assert torch.equal(h2[[0, 3]], table[[5, 7]]) and not y2[[0, 3]].isnan().any()
    assert not kernels.embed_rmsnorm_fits(torch.zeros(4, 13, device=device, dtype=torch.float16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("n_q,n_kv", [(32, 32), (9, 3)])
def test_rope_append_matches_reference_rope_and_slot_write(device, dtype, n_q, n_kv) -> None:
    d, T, theta, bs, nb = 64, 11, 130000.0, 16, 8
    g = seeded(n_q)
    qkv = torch.randn(T, (n_q + 2 * n_kv) * d, generator=g).to(dtype)
    positions = torch.tensor([0, 1, 5, 17, 300, 301, 4095, 4096, 7000, 7471, 12], dtype=torch.int32)
    perm = torch.randperm(nb * bs, generator=g)[:T]
    slots = perm.to(torch.int32)
    slots[3] = -1  # padding: skipped
    table = RotaryTable(d, theta, 8192, device, dtype)
    kp = torch.zeros(n_kv, nb, bs, d, dtype=dtype, device=device)
    vp = torch.zeros_like(kp)
    q = kernels.rope_append(qkv.to(device), positions.to(device), table.cos, table.sin, n_q, n_kv,
                            d, slots.to(device), kp, vp)
    # The kernel's arithmetic is checked bit for bit on the table's own cos/sin values; the table
    # against the reference's per-step cos/sin within a few ulp (torch's CPU cos differs by an
    # ulp between vectorised and scalar paths, so the values themselves are not bit-stable).
    cos, sin = table.cos[positions.long()].cpu(), table.sin[positions.long()].cpu()
    ref_cos, ref_sin = om.rope_cos_sin(positions.long(), d, theta, dtype)
    torch.testing.assert_close(cos.float(), ref_cos.float(), rtol=0, atol=2e-3 if dtype == torch.float16 else 1e-6)
    torch.testing.assert_close(sin.float(), ref_sin.float(), rtol=0, atol=2e-3 if dtype == torch.float16 else 1e-6)
    heads = qkv.view(T, n_q + 2 * n_kv, d)
    q_ref = om.apply_rope(heads[:, :n_q].transpose(0, 1)[None], cos, sin)[0].transpose(0, 1)
    k_ref = om.apply_rope(heads[:, n_q : n_q + n_kv].transpose(0, 1)[None], cos, sin)[0]
    v_ref = heads[:, n_q + n_kv :].transpose(0, 1)
    assert torch.equal(q.cpu(), q_ref)
    kc, vc = kp.cpu(), vp.cpu()
    for t in range(T):
        s = int(slots[t])
        if s < 0:
            continue
        assert torch.equal(kc[:, s // bs, s % bs], k_ref[:, t])
        assert torch.equal(vc[:, s // bs, s % bs], v_ref[:, t])
    written = np.zeros((nb, bs), bool)
    for s in slots.tolist():
        if s >= 0:
            written[s // bs, s % bs] = True
    assert float(kc[:, ~written].abs().sum()) == 0.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_silu_mul(device, dtype) -> None:
    g = seeded(7)
    gu = (torch.randn(9, 2 * 8192, generator=g) * 3).to(dtype)
    out = kernels.silu_mul(gu.to(device), 8192).cpu()
    ref = F.silu(gu[:, :8192]) * gu[:, 8192:]
    if dtype == torch.float32:
        torch.testing.assert_close(out, ref, rtol=1e-6, atol=1e-6)
    else:
        torch.testing.assert_close(out.float(), ref.float(), rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,cols", [(1, 49152), (8, 49152), (64, 49152), (5, 1000), (3, 7),
                                       (4, 70000)])
def test_argmax_rows_is_torch_argmax(device, dtype, rows, cols) -> None:
    """The greedy choice over logit rows equals torch.argmax (the first index of the maximum),
    including planted ties, -inf rows, NaN, a maximum in the last element, and strided rows."""
    g = seeded(rows * 7 + cols)
    x = torch.randn(rows, cols + 16, generator=g).to(dtype)
    if cols > 10:
        x[0, cols // 3] = x[0, cols // 2] = 50.0  # tie: the first index wins
    if rows > 1:
        x[1, :] = float("-inf")
        x[1, cols - 1] = float("-inf")  # all -inf: index 0
    if rows > 2:
        x[2, cols - 1] = 60.0  # the last element
    if rows > 3:
        x[3, 5] = float("nan")
        x[3, 2] = float("nan")  # NaN counts as the maximum; the first one wins
    xd = x.to(device)
    for view in (xd[:, :cols].contiguous(), xd[:, :cols]):  # contiguous, then strided rows
        got = kernels.argmax_rows(view).cpu()
        assert torch.equal(got, x[:, :cols].argmax(dim=-1).to(torch.int32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_positions_outside_the_rope_table_give_nan_not_a_clamp(device, dtype) -> None:
    """A position outside the caller's cos/sin table has no rotation to give: the token's q and k
    come out NaN in both the launch and the per-token rows of the fused projection, while the
    in-table tokens keep their exact values and v is still appended."""
    d, n_q, n_kv, bs, nb, max_pos = 64, 4, 2, 16, 4, 64
    g = seeded(77)
    T = 4
    qkv = torch.randn(T, (n_q + 2 * n_kv) * d, generator=g).to(dtype)
    positions = torch.tensor([3, 64, -1, 63], dtype=torch.int32)  # 64 and -1: no row
    slots = torch.tensor([0, 1, 2, 3], dtype=torch.int32)
    table = RotaryTable(d, 10000.0, max_pos, device, dtype)
    kp = torch.zeros(n_kv, nb, bs, d, dtype=dtype, device=device)
    vp = torch.zeros_like(kp)
    q = kernels.rope_append(qkv.to(device), positions.to(device), table.cos, table.sin, n_q, n_kv,
                            d, slots.to(device), kp, vp).cpu()
    kc, vc = kp.cpu(), vp.cpu()
    heads = qkv.view(T, n_q + 2 * n_kv, d)
    for t, bad in enumerate([False, True, True, False]):
        assert bool(q[t].isnan().all()) == bad and bool(q[t].isnan().any()) == bad
        assert bool(kc[:, 0, t].isnan().all()) == bad and bool(kc[:, 0, t].isnan().any()) == bad
        assert torch.equal(vc[:, 0, t], heads[t, n_q + n_kv :])
    cos_rows, sin_rows = kernels.rope_rows(positions.to(device), table.cos, table.sin)
    assert cos_rows[[1, 2]].isnan().all() and sin_rows[[1, 2]].isnan().all()
    assert torch.equal(cos_rows[[0, 3]], table.cos[[3, 63]])
    assert torch.equal(sin_rows[[0, 3]], table.sin[[3, 63]])
