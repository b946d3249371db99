"""Pins of the quantisation oracle (oracle/quant.py, oracle/c): CPU only.

Known-answer vectors and error bands restate tests/test_quant.py; the torch restatement of
edgerag/core/quant.py is cross-checked byte for byte against the independent C restatement
(plain loops, IEEE rint / division, hand-written fp16 rounding); the linear is checked against
its float64 closed form. Planted mistakes (round-half-away-from-zero, the wrong group axis, the
unbiased nibble) must fail.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import quant as oq
from tests.conftest import seeded


def _weight(n=64, k=256, seed=0):
    return torch.randn(n, k, generator=seeded(seed)) * 0.02


@pytest.mark.parametrize("bits", [1, 3, 16])
def test_config_rejects_bad_widths(bits) -> None:
    with pytest.raises(ValueError, match="only 4- and 8-bit"):
        oq.QuantConfig(bits=bits)


def test_ragged_groups_and_odd_width_rejected() -> None:
    with pytest.raises(ValueError, match="not divisible"):
        oq.quantize_groupwise(_weight(4, 100), oq.QuantConfig(group_size=128))
    with pytest.raises(ValueError, match="must be even"):
        oq.pack_int4(torch.zeros(4, 7, dtype=torch.int8))


def test_known_answer_vectors() -> None:
    """test_quant.py:193-232."""
    codes, scales = oq.quantize_groupwise(torch.zeros(4, 128))
    assert torch.isfinite(scales).all()
    assert torch.equal(oq.dequantize_groupwise(codes, scales), torch.zeros(4, 128).half())
    w = torch.tensor([[float(v) for v in range(-7, 8)] * 8])
    c, s = oq.quantize_groupwise(w, oq.QuantConfig(group_size=120))
    torch.testing.assert_close(oq.dequantize_groupwise(c, s, oq.QuantConfig(120)).float(), w,
                               atol=1e-3, rtol=1e-3)
    kat = torch.tensor([[-7, 7, -1, 1, 0, -4, 4, -7]], dtype=torch.int8)
    assert torch.equal(oq.unpack_int4(oq.pack_int4(kat), 8), kat)
    # byte j = (c[2j] + 8) | (c[2j+1] + 8) << 4, written out for the KAT
    expected = [(a + 8) | ((b + 8) << 4) for a, b in ((-7, 7), (-1, 1), (0, -4), (4, -7))]
    assert oq.pack_int4(kat).tolist() == [expected]
    codes, _ = oq.quantize_groupwise(_weight())
    assert int(codes.max()) <= 7 and int(codes.min()) >= -7
    assert oq.pack_int4(codes).shape == (64, 128)


def test_error_bands_match_4bit_theory() -> None:
    """test_quant.py:87-98."""
    stats = oq.quantization_error(_weight())
    assert 0.05 < stats["relative_error"] < 0.18
    assert stats["signal_to_noise_db"] > 18.0


def test_wrong_axis_is_dramatically_worse() -> None:
    """test_quant.py:101-143 (P-20): a planted transposed grouping must be caught."""
    w = _weight(256, 256) * torch.linspace(0.01, 4.0, 256).unsqueeze(1)
    cfg = oq.QuantConfig()

    def restore(x):
        c, s = oq.quantize_groupwise(x, cfg)
        return oq.dequantize_groupwise(c, s, cfg).float()

    def worst(r):
        return float(((r - w).abs().mean(dim=1) / w.abs().mean(dim=1)).max())

    assert worst(restore(w.T.contiguous()).T.contiguous()) > 5 * worst(restore(w))


@pytest.mark.parametrize("n,k,g,bits", [(64, 256, 128, 4), (33, 120, 120, 4), (40, 512, 512, 8),
                                        (16, 2048, 2048, 8), (8, 1152, 128, 4), (9, 96, 6, 4)])
def test_torch_and_c_restatements_agree_bit_for_bit(n, k, g, bits) -> None:
    w = _weight(n, k, n + k) * (1 + torch.arange(n).unsqueeze(1) % 5)
    cfg = oq.QuantConfig(g, bits)
    codes, scales = oq.quantize_groupwise(w, cfg)
    c_codes, c_scales = c_oracle.quantize(w.numpy(), g, bits)
    assert np.array_equal(codes.numpy(), c_codes)
    assert np.array_equal(scales.numpy().view(np.uint16), c_scales.view(np.uint16))
    if bits == 4:
        assert np.array_equal(oq.pack_int4(codes).numpy(), c_oracle.pack_int4(c_codes))
        assert np.array_equal(c_oracle.unpack_int4(c_oracle.pack_int4(c_codes), k), c_codes)
    deq = oq.dequantize_groupwise(codes, scales, cfg)
    assert np.array_equal(deq.numpy().view(np.uint16),
                          c_oracle.dequantize(c_codes, c_scales, g).view(np.uint16))


def test_ties_round_half_to_even_and_planted_half_away_is_caught() -> None:
    """torch.round is half-to-even (quant.py:94): w / scale = 2.5 must give 2, not 3."""
    w = torch.tensor([[7.0, 2.5, -2.5, 3.5, -0.5, 0.5] + [0.0] * 2])  # amax 7 -> scale 1.0
    codes, scales = oq.quantize_groupwise(w, oq.QuantConfig(group_size=8, bits=4))
    assert float(scales[0, 0]) == 1.0
    assert codes[0, :6].tolist() == [7, 2, -2, 4, 0, 0]
    c_codes, _ = c_oracle.quantize(w.numpy(), 8, 4)
    assert c_codes[0, :6].tolist() == [7, 2, -2, 4, 0, 0]
    planted = torch.floor(w[0, :6] + 0.5).to(torch.int8).tolist()
    assert planted != codes[0, :6].tolist()


def test_dequantize_product_rounds_once_in_fp16() -> None:
    """quant.py:106-107: fp16(code) * fp16(scale) rounds the exact product once."""
    codes = torch.tensor([[127, -127, 3, 0]], dtype=torch.int8)
    scales = torch.tensor([[0.0001234]], dtype=torch.float16)
    out = oq.dequantize_groupwise(codes, scales, oq.QuantConfig(group_size=4, bits=8))
    exact = codes.double() * scales.double()
    assert torch.equal(out, exact.half())


@pytest.mark.parametrize("m", [1, 8, 64])
def test_quant_linear_reference_equals_float64_closed_form(m) -> None:
    cfg = oq.QuantConfig(128, 4)
    w = _weight(48, 256, m)
    packed, scales = oq.quantize_for_layer(w, cfg)
    x = torch.randn(m, 256, generator=seeded(m)).half()
    bias = torch.randn(48, generator=seeded(1)).half()
    ref = oq.quant_linear_reference(x, packed, scales, bias, 256, cfg)
    f64 = oq.quant_linear_f64(x, packed, scales, bias, 256, cfg)
    torch.testing.assert_close(ref.double(), f64, rtol=1e-5, atol=1e-5)
    # a planted unbiased nibble (codes read as 0..15) is far off
    wrong = (packed & 0x0F).float()
    assert not torch.allclose(F_linear(x.float(), wrong), ref, atol=1e-2)


def F_linear(x, w_low_nibbles):
    return x[:, 0::2] @ w_low_nibbles.T
