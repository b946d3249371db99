"""Group-wise INT4 / INT8 weight quantisation on the HIP device.

Same API and storage format as the reference (``edgerag/core/quant.py:44-138``):
``QuantConfig(group_size, bits)``; ``quantize_groupwise`` -> ``(int8 codes, fp16 scales)``;
``dequantize_groupwise``; ``pack_int4`` / ``unpack_int4`` (biased nibbles, low nibble = even k).

The arithmetic runs in the ``edgerag_quantize`` / ``edgerag_dequantize`` kernels and is
bit-identical to the reference: fp32 ``amax / qmax`` scales (1.0 for an all-zero group),
round-half-even codes clamped to ``+-qmax``, fp16 dequantize products. The pack/unpack helpers
are byte shuffles expressed as device tensor ops.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from edgerag_amd import kernels

DEFAULT_GROUP_SIZE = 128
INT4_MAX = 7


@dataclass(frozen=True)
class QuantConfig:
    group_size: int = DEFAULT_GROUP_SIZE
    bits: int = 4

    def __post_init__(self) -> None:
        if self.bits not in (4, 8):
            raise ValueError(f"only 4- and 8-bit are supported, got {self.bits}")
        if self.group_size <= 0:
            raise ValueError(f"group_size must be positive, got {self.group_size}")

    @property
    def qmax(self) -> int:
        return INT4_MAX if self.bits == 4 else 127

    @classmethod
    def per_channel_int8(cls, in_features: int) -> QuantConfig:
        """INT8 with one scale per output channel: ``group_size = in_features``."""
        return cls(group_size=in_features, bits=8)


def _check(weight: torch.Tensor, config: QuantConfig) -> None:
    if weight.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(weight.shape)}")
    if weight.shape[1] % config.group_size:
        raise ValueError(
            f"in_features={weight.shape[1]} is not divisible by group_size={config.group_size}; "
            "a ragged final group would need its own scale and is not supported"
        )


def quantize_packed(weight: torch.Tensor, config: QuantConfig) -> tuple[torch.Tensor, torch.Tensor]:
    """``(packed uint8, scales fp16)`` straight from the kernel: the QuantLinear buffers."""
    _check(weight, config)
    return kernels.quantize(weight, config.bits, config.group_size)


def quantize_groupwise(
    weight: torch.Tensor, config: QuantConfig | None = None
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(codes int8 (N, K), scales fp16 (N, K/g))`` -- the reference return convention."""
    config = config or QuantConfig()
    _check(weight, config)
    # INT8 storage is the codes' two's-complement bytes; for INT4 quantise at 8-bit *storage*
    # would change qmax, so unpack the kernel's packed output instead.
    packed, scales = kernels.quantize(weight, config.bits, config.group_size)
    if config.bits == 8:
        return packed.view(torch.int8), scales
    return unpack_int4(packed, weight.shape[1]), scales


def dequantize_groupwise(
    codes: torch.Tensor, scales: torch.Tensor, config: QuantConfig | None = None
) -> torch.Tensor:
    """fp16 weight from int8 codes and per-group scales."""
    config = config or QuantConfig()
    n, k = codes.shape
    packed = codes.to(torch.int8).view(torch.uint8).contiguous()
    return kernels.dequantize(packed, scales, k, 8, config.group_size)


def pack_int4(codes: torch.Tensor) -> torch.Tensor:
    """Biased nibbles, two per byte along K (low nibble = even k). Device tensors only."""
    kernels.require_device(codes)
    if codes.shape[-1] % 2:
        raise ValueError(f"input dimension {codes.shape[-1]} must be even to pack two per byte")
    biased = (codes.to(torch.int16) + 8).clamp(0, 15).to(torch.uint8)
    return (biased[..., 0::2] | (biased[..., 1::2] << 4)).contiguous()


def unpack_int4(packed: torch.Tensor, in_features: int) -> torch.Tensor:
    """Inverse of :func:`pack_int4`, signed int8 codes. Device tensors only."""
    kernels.require_device(packed)
    low = (packed & 0x0F).to(torch.int16) - 8
    high = ((packed >> 4) & 0x0F).to(torch.int16) - 8
    return torch.stack((low, high), dim=-1).reshape(*packed.shape[:-1], in_features).to(torch.int8)
