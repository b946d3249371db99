"""Oracle for weight-only INT8 / INT4 quantisation and the quant linear (test infrastructure only).

Restates ``edgerag/core/quant.py`` and ``QuantLinear`` (``edgerag/core/linear.py:107-215``) in
torch CPU with the same operations in the same order, so ``torch.round`` (half-to-even), the fp32
scale division and the fp16 dequantize product are the reference's own.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

INT4_MAX = 7


@dataclass(frozen=True)
class QuantConfig:
    """quant.py:44-57."""

    group_size: int = 128
    bits: int = 4

    def __post_init__(self) -> None:
        if self.bits not in (4, 8):
            raise ValueError(f"only 4- and 8-bit are supported, got {self.bits}")
        if self.group_size <= 0:
            raise ValueError(f"group_size must be positive, got {self.group_size}")

    @property
    def qmax(self) -> int:
        return INT4_MAX if self.bits == 4 else 127


def quantize_groupwise(weight: torch.Tensor, config: QuantConfig | None = None):
    """quant.py:60-95 -> ``(codes int8 (N, K), scales fp16 (N, K/g))``."""
    config = config or QuantConfig()
    if weight.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(weight.shape)}")
    n, k = weight.shape
    if k % config.group_size:
        raise ValueError(
            f"in_features={k} is not divisible by group_size={config.group_size}"
        )
    grouped = weight.detach().float().reshape(n, k // config.group_size, config.group_size)
    amax = grouped.abs().amax(dim=-1, keepdim=True)
    scales = torch.where(amax > 0, amax / config.qmax, torch.ones_like(amax))
    codes = torch.round(grouped / scales).clamp(-config.qmax, config.qmax).to(torch.int8)
    return codes.reshape(n, k), scales.squeeze(-1).half()


def dequantize_groupwise(codes, scales, config: QuantConfig | None = None) -> torch.Tensor:
    """quant.py:98-107: ``codes.half() * scales`` per group, in fp16."""
    config = config or QuantConfig()
    n, k = codes.shape
    grouped = codes.reshape(n, k // config.group_size, config.group_size).to(torch.float16)
    return (grouped * scales.unsqueeze(-1)).reshape(n, k)


def pack_int4(codes: torch.Tensor) -> torch.Tensor:
    """quant.py:110-125: biased nibbles, low nibble = even k."""
    if codes.shape[-1] % 2:
        raise ValueError(f"input dimension {codes.shape[-1]} must be even to pack two per byte")
    biased = (codes.to(torch.int16) + 8).clamp(0, 15).to(torch.uint8)
    return (biased[..., 0::2] | (biased[..., 1::2] << 4)).contiguous()


def unpack_int4(packed: torch.Tensor, in_features: int) -> torch.Tensor:
    """quant.py:128-138."""
    low = (packed & 0x0F).to(torch.int16) - 8
    high = ((packed >> 4) & 0x0F).to(torch.int16) - 8
    out = torch.empty((*packed.shape[:-1], in_features), dtype=torch.int8)
    out[..., 0::2] = low.to(torch.int8)
    out[..., 1::2] = high.to(torch.int8)
    return out


def quantize_for_layer(weight: torch.Tensor, config: QuantConfig):
    """QuantLinear.load_weight, linear.py:178-179 -> ``(packed uint8, scales fp16)``."""
    codes, scales = quantize_groupwise(weight, config)
    packed = pack_int4(codes) if config.bits == 4 else codes.to(torch.uint8)
    return packed, scales


def dequantized(packed: torch.Tensor, scales: torch.Tensor, in_features: int,
                config: QuantConfig) -> torch.Tensor:
    """QuantLinear.dequantized, linear.py:186-192."""
    codes = unpack_int4(packed, in_features) if config.bits == 4 else packed.to(torch.int8)
    return dequantize_groupwise(codes, scales, config)


def quant_linear_reference(x, packed, scales, bias, in_features, config) -> torch.Tensor:
    """QuantLinear.forward, linear.py:194-196, evaluated in fp32 from the fp16 weight.

    The reference runs ``F.linear`` in fp16 on the GPU; the fp32 evaluation of the same fp16
    operands is the value both sides approximate, so it is what the kernel is checked against.
    """
    w = dequantized(packed, scales, in_features, config).float()
    b = bias.float() if bias is not None else None
    return F.linear(x.float(), w, b)


def quant_linear_f64(x, packed, scales, bias, in_features, config) -> torch.Tensor:
    """Closed form ``y = x . fp16(code * scale)^T (+ b)`` accumulated in float64."""
    w = dequantized(packed, scales, in_features, config).double()
    y = x.double() @ w.T
    if bias is not None:
        y = y + bias.double()
    return y


def quantization_error(weight: torch.Tensor, config: QuantConfig | None = None) -> dict[str, float]:
    """quant.py:141-176."""
    config = config or QuantConfig()
    codes, scales = quantize_groupwise(weight, config)
    restored = dequantize_groupwise(codes, scales, config).float()
    original = weight.detach().float()
    error = (restored - original).abs()
    denom = original.abs().mean().clamp(min=1e-12)
    row_rel = error.mean(dim=1) / original.abs().mean(dim=1).clamp(min=1e-12)
    return {
        "max_abs_error": float(error.max()),
        "mean_abs_error": float(error.mean()),
        "relative_error": float(error.mean() / denom),
        "max_row_relative_error": float(row_rel.max()),
        "signal_to_noise_db": float(
            10 * torch.log10(
                original.pow(2).mean() / (restored - original).pow(2).mean().clamp(min=1e-20)
            )
        ),
    }
