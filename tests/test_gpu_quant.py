"""INT8 / INT4 quantisation and quant linear on the GPU against the oracle.

Bit-exact: quantize (codes + fp16 scales), pack, dequantize. Within fp16 rtol 1e-2 (north_star):
the fused linear against dequant-then-matmul evaluated in fp32 on the same fp16 weights.
Shapes are BASELINE config 4; KATs restate tests/test_quant.py.
"""

from __future__ import annotations

import pytest
import torch

from edgerag_amd import kernels
from edgerag_amd.core.linear import FP16Linear, QuantLinear
from edgerag_amd.core.quant import (
    QuantConfig,
    dequantize_groupwise,
    pack_int4,
    quantize_groupwise,
    unpack_int4,
)
from oracle import quant as oq
from tests.conftest import seeded

pytestmark = pytest.mark.gpu

LINEAR_TOL = dict(rtol=1e-2, atol=2e-3)

CFG4 = [  # (K, N, bits, group) -- INT8 per-channel and INT4 g128
    (2048, 2048, 8, 2048),
    (2048, 8192, 8, 2048),
    (8192, 2048, 8, 8192),
    (1152, 1152, 4, 128),
    (1152, 4608, 4, 128),
]


def _weight(n, k, seed, scale=0.02, dtype=torch.float16):
    return (torch.randn(n, k, generator=seeded(seed)) * scale).to(dtype)


@pytest.mark.parametrize(
    "n,k,bits,g,dtype",
    [
        (64, 256, 4, 128, torch.float32),
        (64, 256, 8, 128, torch.float32),
        (64, 256, 8, 256, torch.float16),
        (33, 120, 4, 120, torch.float32),
        (17, 96, 4, 6, torch.bfloat16),
        *[(n, k, b, g, torch.float16) for (k, n, b, g) in CFG4],
    ],
)
def test_quantize_is_bit_exact(device, n, k, bits, g, dtype) -> None:
    w = _weight(n, k, n * 7 + k, dtype=dtype)
    cfg = oq.QuantConfig(group_size=g, bits=bits)
    exp_packed, exp_scales = oq.quantize_for_layer(w, cfg)
    packed, scales = kernels.quantize(w.to(device), bits, g)
    assert torch.equal(packed.cpu(), exp_packed)
    assert torch.equal(scales.cpu().view(torch.int16), exp_scales.view(torch.int16))
    codes, sc = quantize_groupwise(w.to(device), QuantConfig(g, bits))
    exp_codes, _ = oq.quantize_groupwise(w, cfg)
    assert torch.equal(codes.cpu(), exp_codes)


@pytest.mark.parametrize("n,k,bits,g", [(64, 256, 4, 128), (40, 512, 8, 512), (16, 1152, 4, 128)])
def test_dequantize_is_bit_exact(device, n, k, bits, g) -> None:
    w = _weight(n, k, 3)
    cfg = oq.QuantConfig(g, bits)
    packed, scales = oq.quantize_for_layer(w, cfg)
    expected = oq.dequantized(packed, scales, k, cfg)
    got = kernels.dequantize(packed.to(device), scales.to(device), k, bits, g)
    assert torch.equal(got.cpu().view(torch.int16), expected.view(torch.int16))


def test_known_answer_vectors(device) -> None:
    """tests/test_quant.py:193-232: zero group, exactly representable levels, nibble signs."""
    codes, scales = quantize_groupwise(torch.zeros(4, 128, device=device), QuantConfig())
    assert torch.isfinite(scales).all()
    assert torch.equal(dequantize_groupwise(codes, scales).cpu(), torch.zeros(4, 128).half())

    w = torch.tensor([[float(v) for v in range(-7, 8)] * 8], device=device)
    c, s = quantize_groupwise(w, QuantConfig(group_size=120))
    torch.testing.assert_close(dequantize_groupwise(c, s, QuantConfig(120)).float(), w,
                               atol=1e-3, rtol=1e-3)

    kat = torch.tensor([[-7, 7, -1, 1, 0, -4, 4, -7]], dtype=torch.int8, device=device)
    assert torch.equal(unpack_int4(pack_int4(kat), 8), kat)
    assert torch.equal(pack_int4(kat).cpu(), oq.pack_int4(kat.cpu()))


@pytest.mark.parametrize("k,n,bits,g", CFG4)
@pytest.mark.parametrize("m", [1, 8, 32, 64, 512, 544])
def test_quant_linear_cfg4(device, k, n, bits, g, m) -> None:
    w = _weight(n, k, k + n)
    cfg = oq.QuantConfig(g, bits)
    packed, scales = oq.quantize_for_layer(w, cfg)
    x = torch.randn(m, k, generator=seeded(m)).half()
    expected = oq.quant_linear_reference(x, packed, scales, None, k, cfg)
    y = kernels.quant_linear(x.to(device), packed.to(device), scales.to(device), None, k, n, bits, g)
    assert y.dtype == torch.float16 and y.shape == (m, n)
    torch.testing.assert_close(y.float().cpu(), expected, **LINEAR_TOL)


@pytest.mark.parametrize("m", [1, 3, 7])
def test_quant_linear_bias_fp32_and_generic_shapes(device, m) -> None:
    """Bias, fp32 activations, and K / group sizes off the vector path (K=120, g=120; g=6)."""
    for (n, k, bits, g, xdt) in [(64, 256, 4, 128, torch.float32), (33, 120, 8, 120, torch.float16),
                                 (19, 96, 4, 6, torch.float16), (48, 512, 8, 512, torch.float32)]:
        w = _weight(n, k, n + k + m)
        cfg = oq.QuantConfig(g, bits)
        packed, scales = oq.quantize_for_layer(w, cfg)
        bias = (torch.randn(n, generator=seeded(n)) * 0.1).half()
        x = torch.randn(m, k, generator=seeded(m + 1)).to(xdt)
        expected = oq.quant_linear_reference(x, packed, scales, bias, k, cfg)
        y = kernels.quant_linear(x.to(device), packed.to(device), scales.to(device),
                                 bias.to(device), k, n, bits, g)
        assert y.dtype == xdt
        tol = LINEAR_TOL if xdt == torch.float16 else dict(rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(y.float().cpu(), expected, **tol)


def test_quant_linear_module_matches_fp16_within_quantization_error(device) -> None:
    """tests/test_quant.py:243-257 on the device module."""
    w = (torch.randn(64, 256, generator=seeded(0)) * 0.02)
    x = torch.randn(4, 256, generator=seeded(7)).half().to(device)
    ref = FP16Linear(256, 64).half().to(device)
    ref.load_weight(w.half().to(device))
    layer = QuantLinear(256, 64, device=device)
    layer.load_weight(w)
    rel = (layer(x).float() - ref(x).float()).abs().mean() / ref(x).float().abs().mean()
    assert float(rel) < 0.12
    before = layer.packed.clone()
    layer(x)
    assert torch.equal(layer.packed, before)  # quantisation happens at load, not in forward
    assert layer.weight_bytes() == 64 * 128 + 64 * 2 * 2


def test_fused_concat_equals_separate_layers(device) -> None:
    layers = []
    for i, n in enumerate((64, 32, 32)):
        layer = QuantLinear(256, n, config=QuantConfig(256, 8), device=device)
        layer.load_weight(torch.randn(n, 256, generator=seeded(i)) * 0.02)
        layers.append(layer)
    fused = QuantLinear.concat(layers)
    x = torch.randn(5, 256, generator=seeded(9)).half().to(device)
    assert torch.equal(fused(x), torch.cat([layer(x) for layer in layers], dim=-1))


@pytest.mark.parametrize("bits,k,g", [(8, 256, 256), (8, 512, 64), (4, 256, 128), (4, 1152, 32)])
@pytest.mark.parametrize("m", [1, 2, 5, 16, 17, 31, 32, 33, 63, 64, 65, 100, 130])
def test_quant_linear_mfma_edges(device, bits, k, g, m) -> None:
    """Both MFMA paths (M <= 32 streaming, M > 32 tiled) on ragged M, N not a multiple of any
    tile (37, 200), bias, and K / group sizes that exercise per-group scales."""
    for n in (37, 200):
        w = _weight(n, k, n * 3 + k + bits)
        cfg = oq.QuantConfig(g, bits)
        packed, scales = oq.quantize_for_layer(w, cfg)
        bias = (torch.randn(n, generator=seeded(n + m)) * 0.1).half()
        x = torch.randn(m, k, generator=seeded(m * 11 + n)).half()
        expected = oq.quant_linear_reference(x, packed, scales, bias, k, cfg)
        y = kernels.quant_linear(x.to(device), packed.to(device), scales.to(device),
                                 bias.to(device), k, n, bits, g)
        torch.testing.assert_close(y.float().cpu(), expected, **LINEAR_TOL)


@pytest.mark.parametrize("k,n", [(2048, 16384), (640, 8200), (1152, 8192)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_quant_linear_swiglu_fused(device, k, n, with_bias) -> None:
    """SwiGLU in the streaming GEMV's epilogue (decode batches, [gate; up] INT8 per-channel):
    bit-identical to the projection followed by silu_mul for M = 1..64 (one launch against two),
    and within the linear tolerance of silu(gate) * up from the oracle's dequant-then-matmul.
    K a whole number of per-wave batches (2048) and not (640, 1152); I = N / 2 not a multiple of
    the 16-row tile (4100); strided activations."""
    w = _weight(n, k, n + 3 * k)
    cfg = oq.QuantConfig(k, 8)
    packed, scales = oq.quantize_for_layer(w, cfg)
    bias = (torch.randn(n, generator=seeded(n - k)) * 0.1).half() if with_bias else None
    inter = n // 2
    pd, sd = packed.to(device), scales.to(device)
    bd = bias.to(device) if bias is not None else None
    for m in (1, 3, 8, 16, 17, 32, 40, 64):
        assert kernels.quant_swiglu_fused(m, k, n, 8, k)
        xfull = torch.randn(m, k + 64, generator=seeded(m * 29 + k)).half()
        xd = xfull.to(device)[:, :k]
        fused = kernels.quant_linear_swiglu(xd, pd, sd, bd, k, n, 8, k)
        gu = kernels.quant_linear(xd, pd, sd, bd, k, n, 8, k, split_k=False)
        plain = kernels.silu_mul(gu, inter)
        assert fused.shape == (m, inter)
        assert torch.equal(fused, plain), f"M={m}: fused SwiGLU differs from projection + silu_mul"
        ref_gu = oq.quant_linear_reference(xfull[:, :k], packed, scales, bias, k, cfg)
        ref = torch.nn.functional.silu(ref_gu[:, :inter]) * ref_gu[:, inter:]
        torch.testing.assert_close(fused.float().cpu(), ref, **LINEAR_TOL)


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Equal values, NaN matching NaN (positions outside the RoPE table)."""
    return bool(((a == b) | (a.isnan() & b.isnan())).all()) and a.shape == b.shape


@pytest.mark.parametrize("n_q,n_kv,d,k", [(32, 32, 64, 2048), (32, 8, 128, 1024),
                                           (16, 4, 64, 640)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_quant_linear_rope_append_fused(device, n_q, n_kv, d, k, with_bias) -> None:
    """q/k/v projection + RoPE + KV append in the streaming GEMV's epilogue: q_out and both pools
    bit-identical to quant_linear followed by rope_append, for decode batches (M <= 16) and
    M up to 64; GQA and head_dim 128 (four workgroups per head); slots that are padding (-1) or
    past the pool leave the pools untouched. Shapes whose plain launch uses two k-slices (N < 4096
    at M <= 32) take the two-launch path through the same entry."""
    from edgerag_amd.core.layers import RotaryTable

    n = (n_q + 2 * n_kv) * d
    w = _weight(n, k, n + k + d)
    cfg = oq.QuantConfig(k, 8)
    packed, scales = oq.quantize_for_layer(w, cfg)
    bias = (torch.randn(n, generator=seeded(n + 1)) * 0.1).half() if with_bias else None
    pd, sd = packed.to(device), scales.to(device)
    bd = bias.to(device) if bias is not None else None
    bs, nb = 16, 64
    table = RotaryTable(d, 130000.0, 8192, device, torch.float16)
    for m in (1, 3, 8, 16, 17, 33, 64):
        g = seeded(m * 7 + d)
        x = torch.randn(m, k, generator=g).half().to(device)
        # Some positions past the 8192-row table: NaN q and k on both paths.
        positions = torch.randint(0, 9000, (m,), generator=g, dtype=torch.int32)
        slots = torch.randperm(nb * bs, generator=g)[:m].to(torch.int32)
        slots[0] = -1
        if m > 2:
            slots[2] = nb * bs + 5
        pos_d, slots_d = positions.to(device), slots.to(device)
        rows = kernels.rope_rows(pos_d, table.cos, table.sin)
        fused = kernels.quant_rope_fused(m, k, 8, k, n_q, n_kv, d)
        if n >= 4096:  # the plain projection streams with one k-slice: fused
            assert fused
        pools = []
        qs = []
        for use_rows in (rows, None):  # fused launch, then the two-launch path
            kp = torch.full((n_kv, nb, bs, d), 7.0, dtype=torch.float16, device=device)
            vp = torch.full_like(kp, -3.0)
            q = kernels.quant_linear_rope_append(
                x, pd, sd, bd, k, 8, k, pos_d, table.cos, table.sin, n_q, n_kv, d, slots_d, kp, vp,
                rows=use_rows)
            qs.append(q)
            pools.append((kp, vp))
        assert _same(qs[0], qs[1]), f"M={m}: q differs from the two-launch path"
        assert _same(pools[0][0], pools[1][0]), f"M={m}: key pool differs"
        assert torch.equal(pools[0][1], pools[1][1]), f"M={m}: value pool differs"
        past = positions.to(device) >= 8192
        assert bool(qs[0][past].isnan().all()) and not bool(qs[0][~past].isnan().any())
        # Padding and out-of-pool slots wrote nothing; every valid slot was written.
        kc = pools[0][0].cpu()
        valid = [int(s) for s in slots if 0 <= int(s) < nb * bs]
        for s_ in valid:
            assert not torch.all(kc[:, s_ // bs, s_ % bs] == 7.0)
        untouched = torch.ones(nb * bs, dtype=torch.bool)
        untouched[valid] = False
        assert torch.all(kc.reshape(n_kv, nb * bs, d)[:, untouched] == 7.0)


@pytest.mark.parametrize("n_q,n_kv,k,ms", [
    (32, 32, 2048, (384, 512, 519, 544)),  # config 5's q/k/v: 128x64 tiles
    (48, 16, 2048, (512, 519)),            # GQA: q / k / v boundaries between workgroups' heads
    (64, 64, 1024, (200, 512, 519, 544)),  # 128x128 tiles from M = 257; M = 519 streams 7 rows
])
def test_quant_linear_rope_append_tiled_gemm(device, n_q, n_kv, k, ms) -> None:
    """q/k/v projection + RoPE + KV append in the tiled GEMM's epilogue (prefill slices, M > 64,
    head_dim 64, weights whose plain launch takes 128-row tiles): each wave's 64 rows are one
    head, so every rotate_half partner is in the same lane. q_out and both pools bit-identical to
    quant_linear followed by rope_append; padding and out-of-pool slots leave the pools alone."""
    from edgerag_amd.core.layers import RotaryTable

    d = 64
    n = (n_q + 2 * n_kv) * d
    w = _weight(n, k, n + 3 * k)
    cfg = oq.QuantConfig(k, 8)
    packed, scales = oq.quantize_for_layer(w, cfg)
    bias = (torch.randn(n, generator=seeded(n + 3)) * 0.1).half()
    pd, sd, bd = packed.to(device), scales.to(device), bias.to(device)
    bs, nb = 16, 64
    table = RotaryTable(d, 130000.0, 8192, device, torch.float16)
    for m in ms:
        assert kernels.quant_rope_fused(m, k, 8, k, n_q, n_kv, d), f"M={m}"
        g = seeded(m * 11 + n_q)
        x = torch.randn(m, k, generator=g).half().to(device)
        positions = torch.randint(0, 8192, (m,), generator=g, dtype=torch.int32)
        slots = torch.randperm(nb * bs, generator=g)[:m].to(torch.int32)
        slots[0] = -1
        slots[m - 1] = nb * bs + 5  # past the pool (a remainder row at M = 519)
        pos_d, slots_d = positions.to(device), slots.to(device)
        rows = kernels.rope_rows(pos_d, table.cos, table.sin)
        pools, qs = [], []
        for use_rows in (rows, None):  # fused launch, then the two-launch path
            kp = torch.full((n_kv, nb, bs, d), 7.0, dtype=torch.float16, device=device)
            vp = torch.full_like(kp, -3.0)
            q = kernels.quant_linear_rope_append(
                x, pd, sd, bd, k, 8, k, pos_d, table.cos, table.sin, n_q, n_kv, d, slots_d, kp, vp,
                rows=use_rows)
            qs.append(q)
            pools.append((kp, vp))
        assert torch.equal(qs[0], qs[1]), f"M={m}: q differs from the two-launch path"
        assert torch.equal(pools[0][0], pools[1][0]), f"M={m}: key pool differs"
        assert torch.equal(pools[0][1], pools[1][1]), f"M={m}: value pool differs"
        vc = pools[0][1].cpu()
        valid = [int(s_) for s_ in slots if 0 <= int(s_) < nb * bs]
        untouched = torch.ones(nb * bs, dtype=torch.bool)
        untouched[valid] = False
        assert torch.all(vc.reshape(n_kv, nb * bs, d)[:, untouched] == -3.0)


@pytest.mark.parametrize("k,n,ms", [
    (2048, 16384, (65, 128, 200, 512, 519, 544)),
    (2048, 6144, (384, 512, 519, 544)),   # 128x64 tiles from 6 tile rows (M > 320) on
    (1152, 8192, (320, 512, 519, 544)),
    (1024, 8200, (512, 519)),  # I = 4100: the last 64-column block holds 4 outputs
])
def test_quant_linear_swiglu_tiled_gemm(device, k, n, ms) -> None:
    """SwiGLU in the tiled GEMM's epilogue (prefill slices, M > 64, weights whose plain launch
    takes 128-row tiles: 128x128 for 2048 -> 16384 and 1152 -> 8192 at M = 512, 128x64 for
    2048 -> 6144): bit-identical to the projection followed by silu_mul, including M = 519
    (512 chunk tokens + 7 decode rows: the remainder on the streaming SwiGLU kernel where the
    plain launch streams it too) and M = 544; within the linear tolerance of the oracle."""
    w = _weight(n, k, n + 5 * k)
    cfg = oq.QuantConfig(k, 8)
    packed, scales = oq.quantize_for_layer(w, cfg)
    bias = (torch.randn(n, generator=seeded(n + k)) * 0.1).half()
    inter = n // 2
    pd, sd, bd = packed.to(device), scales.to(device), bias.to(device)
    for m in ms:
        assert kernels.quant_swiglu_fused(m, k, n, 8, k)
        x = torch.randn(m, k, generator=seeded(m * 31 + k)).half()
        xd = x.to(device)
        fused = kernels.quant_linear_swiglu(xd, pd, sd, bd, k, n, 8, k)
        gu = kernels.quant_linear(xd, pd, sd, bd, k, n, 8, k, split_k=False)
        plain = kernels.silu_mul(gu, inter)
        assert fused.shape == (m, inter)
        assert torch.equal(fused, plain), f"M={m}: fused SwiGLU differs from projection + silu_mul"
        if m == ms[0]:
            ref_gu = oq.quant_linear_reference(x, packed, scales, bias, k, cfg)
            ref = torch.nn.functional.silu(ref_gu[:, :inter]) * ref_gu[:, inter:]
            torch.testing.assert_close(fused.float().cpu(), ref, **LINEAR_TOL)


def test_quant_linear_swiglu_falls_back_outside_its_shapes(device) -> None:
    """Shapes the fused launch does not cover (M > 64 on a weight whose plain launch takes
    64x64 tiles, N below two tiles per workgroup, INT4) run as projection + silu_mul through the
    same entry, and the C entry point says why."""
    k, n = 1024, 2048
    w = _weight(n, k, 77)
    for bits, g, m in ((8, k, 4), (8, k, 80), (4, 128, 4)):
        cfg = oq.QuantConfig(g, bits)
        packed, scales = oq.quantize_for_layer(w, cfg)
        assert not kernels.quant_swiglu_fused(m, k, n, bits, g)
        x = torch.randn(m, k, generator=seeded(m + bits)).half().to(device)
        pd, sd = packed.to(device), scales.to(device)
        y = kernels.quant_linear_swiglu(x, pd, sd, None, k, n, bits, g)
        gu = kernels.quant_linear(x, pd, sd, None, k, n, bits, g, split_k=False)
        assert torch.equal(y, kernels.silu_mul(gu, n // 2))
    with pytest.raises(kernels._lib.EdgeragError, match="not covered"):
        kernels.call("edgerag_quant_linear_swiglu", x.data_ptr(), 1, k, 4, k, pd.data_ptr(),
                     sd.data_ptr(), None, n, 4, 128, y.data_ptr(), n // 2, None, 0, 0.0,
                     kernels.stream_ptr(x.device))


@pytest.mark.parametrize("k,n", [(2048, 2048), (8192, 2048), (2048, 4096), (2048, 8192),
                                 (640, 1004)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_quant_linear_residual(device, k, n, with_bias) -> None:
    """The residual producer (decode batches): hidden becomes fp16(hidden + y) bit for bit, with y
    exactly the plain launch's output, xw = fp16(w * hidden) bit for bit, and the per-workgroup
    partials sum to the new rows' sum of squares. Shapes cover 8-row tiles (two k-slices), 16-row and two-tile workgroups, and a last
    workgroup with fewer rows than its tile (N 1004)."""
    w = _weight(n, k, n * 3 + k)
    cfg = oq.QuantConfig(k, 8)
    packed, scales = oq.quantize_for_layer(w, cfg)
    bias = (torch.randn(n, generator=seeded(n + 5)) * 0.1).half() if with_bias else None
    pd, sd = packed.to(device), scales.to(device)
    bd = bias.to(device) if bias is not None else None
    for m in (1, 3, 8, 16):
        parts = kernels.quant_residual_parts(m, k, n, 8, k)
        assert parts > 0
        g = seeded(m + k + n)
        x = torch.randn(m, k, generator=g).half().to(device)
        hidden0 = (torch.randn(m, n, generator=g) * 4).half()
        y = kernels.quant_linear(x, pd, sd, bd, k, n, 8, k, split_k=False).cpu()
        expected = (hidden0.float() + y.float()).half()
        hidden = hidden0.to(device)
        partials = torch.full((m * parts,), float("nan"), dtype=torch.float32, device=device)
        nw = (1.0 + 0.3 * torch.randn(n, generator=g)).half()
        xw = torch.full((m, n), float("nan"), dtype=torch.float16, device=device)
        got = kernels.quant_linear_residual(x, pd, sd, bd, k, n, 8, k, hidden, partials,
                                            nw.to(device), xw)
        assert got == parts
        assert torch.equal(hidden.cpu(), expected), f"M={m}: residual add differs"
        assert torch.equal(xw.cpu(), (nw.float() * expected.float()).half())
        ss = partials.view(m, parts).double().cpu().sum(1)
        torch.testing.assert_close(ss, expected.double().pow(2).sum(1), rtol=1e-5, atol=1e-6)
    assert kernels.quant_residual_parts(17, k, n, 8, k) == 0


def _partials_of(h: torch.Tensor, parts: int) -> torch.Tensor:
    """Sums of squares of h's rows over `parts` contiguous column ranges, (M * parts,) fp32."""
    m, k = h.shape
    edges = torch.linspace(0, k, parts + 1).round().long()
    hf = h.float()
    cols = [hf[:, int(edges[p]):int(edges[p + 1])].pow(2).sum(1) for p in range(parts)]
    return torch.stack(cols, 1).reshape(-1).contiguous()


@pytest.mark.parametrize("parts", [256, 250, 7])
def test_quant_linear_normed_inputs(device, parts) -> None:
    """Normed inputs (decode batches): the fused SwiGLU and q/k/v + RoPE launches given
    xw = fp16(w * h) (the residual producer's output) and the partial sums of squares of h compute
    the projection of RMSNorm(h) -- against the float64 oracle and against the two-launch path (rmsnorm kernel, then
    the plain fused launch) within the linear tolerance. Partial counts: the producers' 256, and
    counts that are not a multiple of the 64 lanes."""
    from edgerag_amd.core.layers import RotaryTable
    from oracle import model as om

    k, eps = 2048, 1e-5
    nw = (1.0 + 0.2 * torch.randn(k, generator=seeded(11))).half()
    nwd = nw.to(device)
    # SwiGLU: [gate; up] of 2 x 8192 rows.
    n = 16384
    wgu = _weight(n, k, 21)
    cfg = oq.QuantConfig(k, 8)
    packed, scales = oq.quantize_for_layer(wgu, cfg)
    pd, sd = packed.to(device), scales.to(device)
    for m in (1, 5, 8, 16):
        h = (torch.randn(m, k, generator=seeded(m * 3 + parts)) * 3).half()
        hd = h.to(device)
        part = _partials_of(h, parts).to(device)
        xw = (nw.float() * h.float()).half().to(device)  # what the residual producer writes
        normed = kernels.NormedInput(part, parts, eps)
        got = kernels.quant_linear_swiglu(xw, pd, sd, None, k, n, 8, k, norm=normed).float().cpu()
        xn = om.rms_norm(h, nw, eps)
        ref_gu = oq.quant_linear_reference(xn, packed, scales, None, k, cfg)
        ref = torch.nn.functional.silu(ref_gu[:, : n // 2]) * ref_gu[:, n // 2 :]
        two = kernels.quant_linear_swiglu(kernels.rmsnorm(hd, nwd, eps), pd, sd, None, k, n, 8,
                                          k).float().cpu()
        # silu(g) * u compounds the linear tolerance of g and u (|u| ~ 1 here). The fused path
        # rounds fp16(w * h) where the reference rounds fp16(w * fp16(h * r)): one moved rounding,
        # which may cost at most twice the two-launch path's error against float64.
        err, err_two = (got - ref).abs(), (two - ref).abs()
        assert float(err.max()) <= max(2 * float(err_two.max()), 4e-3), (
            f"M={m}: max error {float(err.max()):.2e} (two-launch {float(err_two.max()):.2e})")
        assert float(err.mean()) <= 2 * float(err_two.mean()) + 1e-6
        torch.testing.assert_close(got, ref, rtol=1e-2, atol=4e-3)
    # q/k/v + RoPE + KV append: 32 / 32 heads of 64.
    n_q = n_kv = 32
    d = 64
    n = (n_q + 2 * n_kv) * d
    wq = _weight(n, k, 23)
    packed, scales = oq.quantize_for_layer(wq, cfg)
    pd, sd = packed.to(device), scales.to(device)
    table = RotaryTable(d, 130000.0, 8192, device, torch.float16)
    bs, nb = 16, 32
    for m in (1, 8, 16):
        h = (torch.randn(m, k, generator=seeded(m * 5 + parts)) * 3).half()
        hd = h.to(device)
        part = _partials_of(h, parts).to(device)
        xw = (nw.float() * h.float()).half().to(device)
        positions = torch.arange(100, 100 + m, dtype=torch.int32).to(device)
        slots = torch.randperm(nb * bs, generator=seeded(m))[:m].to(torch.int32).to(device)
        rows = kernels.rope_rows(positions, table.cos, table.sin)
        outs = []
        for normed in (True, False):
            kp = torch.zeros((n_kv, nb, bs, d), dtype=torch.float16, device=device)
            vp = torch.zeros_like(kp)
            xin = xw if normed else kernels.rmsnorm(hd, nwd, eps)
            norm = kernels.NormedInput(part, parts, eps) if normed else None
            q = kernels.quant_linear_rope_append(
                xin, pd, sd, None, k, 8, k, positions, table.cos, table.sin, n_q, n_kv, d, slots,
                kp, vp, rows=rows, norm=norm)
            outs.append((q.float(), kp.float(), vp.float()))
        for a, b in zip(outs[0], outs[1]):  # rotated q / k and v: linear outputs (|x| ~ 1)
            torch.testing.assert_close(a, b, rtol=1e-2, atol=4e-3)


@pytest.mark.parametrize("k", [640, 1152, 2048, 8192])
@pytest.mark.parametrize("n", [37, 2048, 4104, 8200])
def test_quant_linear_int8_per_channel_streaming(device, k, n) -> None:
    """The per-channel INT8 streaming GEMV (M <= 64): two k-slices per MFMA tile for narrow N,
    one for wide N; K both a whole number of per-wave batches (2048, 8192) and not (640, 1152,
    where the last batch of a wave overlaps the one before); N not a multiple of the row tile;
    bias; activations with a row stride larger than K. The row scale multiplies the fp32 sum,
    so the check is against the reference dequant-then-matmul at the linear tolerance."""
    w = _weight(n, k, n + 7 * k)
    cfg = oq.QuantConfig(k, 8)
    packed, scales = oq.quantize_for_layer(w, cfg)
    bias = (torch.randn(n, generator=seeded(n + k)) * 0.1).half()
    for m in (1, 2, 5, 8, 9, 16, 17, 32, 40, 64):
        xfull = torch.randn(m, k + 64, generator=seeded(m * 13 + k)).half()
        x = xfull[:, :k]
        expected = oq.quant_linear_reference(x, packed, scales, bias, k, cfg)
        y = kernels.quant_linear(xfull.to(device)[:, :k], packed.to(device), scales.to(device),
                                 bias.to(device), k, n, 8, k)
        torch.testing.assert_close(y.float().cpu(), expected, **LINEAR_TOL)
        # Up to 16 tokens (decode batches) the kernel shape depends on N and K only and token
        # rows are independent: each row alone gives the same bits as in the batch.
        if m <= 16:
            y1 = kernels.quant_linear(xfull.to(device)[m - 1 : m, :k], packed.to(device),
                                      scales.to(device), bias.to(device), k, n, 8, k)
            assert torch.equal(y1[0], y[m - 1])


def test_streaming_long_k_rows_independent_of_batch(device) -> None:
    """Two k-slices (N < 4096) over a K long enough that one m-tile alone could take 16 waves:
    the launches of 1..8 and 9..16 tokens split K alike, so every row of a decode batch has the
    bits it has alone, and all match the reference at the linear tolerance."""
    k, n = 16384, 2048
    w = _weight(n, k, 91)
    cfg = oq.QuantConfig(k, 8)
    packed, scales = oq.quantize_for_layer(w, cfg)
    pd, sd = packed.to(device), scales.to(device)
    for m in (8, 9, 16):
        x = torch.randn(m, k, generator=seeded(m + 5)).half()
        xd = x.to(device)
        y = kernels.quant_linear(xd, pd, sd, None, k, n, 8, k)
        torch.testing.assert_close(y.float().cpu(),
                                   oq.quant_linear_reference(x, packed, scales, None, k, cfg),
                                   **LINEAR_TOL)
        for r in (0, m - 1):
            y1 = kernels.quant_linear(xd[r : r + 1], pd, sd, None, k, n, 8, k)
            assert torch.equal(y1[0], y[r])


SPLIT_SHAPES = [  # (K, N, bits, group): 64x64 tile grids below 256 workgroups (the workspace
    # route: unsplit or split K by the cost model)
    (8192, 2048, 8, 8192),
    (2048, 2048, 8, 2048),
    (2048, 8192, 8, 2048),
    (1152, 4608, 4, 128),
    (1152, 1152, 4, 128),
    (512, 200, 8, 64),  # grouped INT8, N off the tile
    (2048, 37, 4, 128),
]


def _split_case(k, n, bits, g, m, seed):
    w = _weight(n, k, seed)
    cfg = oq.QuantConfig(g, bits)
    packed, scales = oq.quantize_for_layer(w, cfg)
    bias = (torch.randn(n, generator=seeded(seed + 1)) * 0.1).half()
    x = torch.randn(m, k, generator=seeded(seed + 2)).half()
    return x, packed, scales, bias, cfg


@pytest.mark.parametrize("k,n,bits,g", SPLIT_SHAPES)
@pytest.mark.parametrize("m", [17, 32, 33, 64, 100, 130])
def test_quant_linear_split_k(device, k, n, bits, g, m) -> None:
    """The workspace route of the tiled GEMM (kernels.quant_linear passes its workspace; split K
    or not) against the oracle's dequant-then-matmul. It is deterministic (partials are added in
    k-range order: two runs give the same bits)."""
    x, packed, scales, bias, cfg = _split_case(k, n, bits, g, m, k + n + m)
    if m >= 33 and (k, n) == (8192, 2048):
        assert kernels.quant_workspace_bytes(m, k, n, bits, g) > 0, "the down projection splits K"
    expected = oq.quant_linear_reference(x, packed, scales, bias, k, cfg)
    args = (packed.to(device), scales.to(device), bias.to(device), k, n, bits, g)
    y1 = kernels.quant_linear(x.to(device), *args)
    y2 = kernels.quant_linear(x.to(device), *args)
    torch.testing.assert_close(y1.float().cpu(), expected, **LINEAR_TOL)
    assert torch.equal(y1, y2)


def test_quant_linear_ws_without_room_is_the_plain_launch(device) -> None:
    """A workspace below the plan's size, unaligned, or none runs edgerag_quant_linear: the same
    bits."""
    from edgerag_amd import _lib

    k, n, bits, g, m = 8192, 2048, 8, 8192, 64
    x, packed, scales, bias, _ = _split_case(k, n, bits, g, m, 3)
    x, packed, scales, bias = (t.to(device) for t in (x, packed, scales, bias))
    need = kernels.quant_workspace_bytes(m, k, n, bits, g)
    assert need > 0
    ws = torch.full((need + 16,), 0xFF, dtype=torch.uint8, device=device)  # any contents
    outs = []
    for name, extra in [("edgerag_quant_linear", ()),
                        ("edgerag_quant_linear_ws", (ws.data_ptr(), need - 1)),
                        ("edgerag_quant_linear_ws", (0, 0)),
                        ("edgerag_quant_linear_ws", (ws.data_ptr() + 4, need)),  # unaligned
                        ("edgerag_quant_linear_ws", (ws.data_ptr(), need))]:
        y = torch.empty(m, n, dtype=torch.float16, device=device)
        _lib.call(name, x.data_ptr(), 1, x.stride(0), m, k, packed.data_ptr(), scales.data_ptr(),
                  bias.data_ptr(), n, bits, g, y.data_ptr(), y.stride(0), *extra,
                  kernels.stream_ptr(device))
        outs.append(y)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    assert torch.equal(outs[0], outs[3])
    torch.testing.assert_close(outs[4].float(), outs[0].float(), **LINEAR_TOL)


def test_quant_linear_split_k_graph_replays(device) -> None:
    """Captured in a HIP graph, the split-K launch replays to the eager bits every time, with
    eager launches that share the workspace between the replays."""
    k, n, bits, g, m = 8192, 2048, 8, 8192, 48
    x, packed, scales, bias, _ = _split_case(k, n, bits, g, m, 5)
    x, packed, scales, bias = (t.to(device) for t in (x, packed, scales, bias))
    x2 = torch.randn(33, 2048, generator=seeded(6)).half().to(device)
    p2, s2 = oq.quantize_for_layer(_weight(2048, 2048, 7), oq.QuantConfig(2048, 8))
    p2, s2 = p2.to(device), s2.to(device)
    eager = kernels.quant_linear(x, packed, scales, bias, k, n, bits, g)
    eager2 = kernels.quant_linear(x2, p2, s2, None, 2048, 2048, 8, 2048)
    out = torch.empty_like(eager)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        kernels.quant_linear(x, packed, scales, bias, k, n, bits, g, out=out)
        with torch.cuda.graph(graph, stream=stream):
            kernels.quant_linear(x, packed, scales, bias, k, n, bits, g, out=out)
    torch.cuda.current_stream(device).wait_stream(stream)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(kernels.quant_linear(x2, p2, s2, None, 2048, 2048, 8, 2048), eager2)


@pytest.mark.parametrize("bits,g,with_bias", [(8, None, False), (4, 128, True), (8, 64, True)])
def test_quant_state_dict_round_trips_through_safetensors(device, tmp_path, bits, g, with_bias):
    """The on-disk quant format: a QuantLinear's state dict (`packed` / `scales` / `bias`, the
    reference's buffers, edgerag/core/linear.py:152-164) saved with safetensors loads into a fresh
    layer without re-quantising (buffers and outputs bit-identical), and a state dict written by
    the oracle's quantiser in the reference layout loads the same way."""
    from safetensors.torch import load_file, save_file

    k, n = 512, 192
    cfg = QuantConfig(g if g is not None else k, bits)
    w = _weight(n, k, 11)
    bias = (torch.randn(n, generator=seeded(12)) * 0.1).half() if with_bias else None
    a = QuantLinear(k, n, bias=with_bias, config=cfg, device=device)
    a.load_weight(w, bias)
    path = tmp_path / "layer.safetensors"
    save_file({key: t.contiguous().cpu() for key, t in a.state_dict().items()}, str(path))
    b = QuantLinear(k, n, bias=with_bias, config=cfg, device=device)
    b.load_state_dict({key: t.to(device) for key, t in load_file(str(path)).items()})
    for key, t in a.state_dict().items():
        assert torch.equal(b.state_dict()[key], t), key
    x = torch.randn(7, k, generator=seeded(13)).half().to(device)
    assert torch.equal(a(x), b(x))
    # A checkpoint quantised elsewhere (the oracle restates the reference's quantiser).
    packed, scales = oq.quantize_for_layer(w, oq.QuantConfig(cfg.group_size, bits))
    ext = {"packed": packed, "scales": scales}
    if with_bias:
        ext["bias"] = bias
    c = QuantLinear(k, n, bias=with_bias, config=cfg, device=device)
    c.load_state_dict({key: t.to(device) for key, t in ext.items()})
    assert torch.equal(c.packed, a.packed) and torch.equal(c.scales, a.scales)
    expected = oq.quant_linear_reference(x.cpu(), packed, scales, bias, k, oq.QuantConfig(cfg.group_size, bits))
    torch.testing.assert_close(c(x).float().cpu(), expected, **LINEAR_TOL)
