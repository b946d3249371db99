"""The linear-layer seam, with weight-only INT8 / INT4 layers on fused HIP kernels.

Mirrors ``edgerag/core/linear.py``: ``LinearBase`` (``forward`` / ``load_weight`` /
``weight_bytes``, ``:44-70``), ``FP16Linear`` (``:73-104``), ``QuantLinear`` with the same buffers
``packed`` uint8 ``(N, K/2 | K)``, ``scales`` fp16 ``(N, K/g)``, optional fp16 ``bias`` (``:152-164``)
and the same errors (``:137-146``, ``:167-176``), plus the skip list (``:229-241``). A reference
state dict therefore loads into this ``QuantLinear`` unchanged.

The difference is ``forward``: the reference dequantizes the whole weight to fp16 and calls
``F.linear`` (``:194-196``), which moves more bytes than the fp16 layer it replaces. Here
``edgerag_quant_linear`` streams the packed bytes once and dequantizes in registers, so INT8 and
INT4 layers read 2x / 4x fewer weight bytes than fp16.
"""

from __future__ import annotations

from abc import abstractmethod
from collections.abc import Callable

import torch
from torch import nn

from edgerag_amd import kernels
from edgerag_amd.core.quant import QuantConfig, quantize_packed

LinearFactory = Callable[..., "LinearBase"]
FP16_BYTES = 2


class LinearBase(nn.Module):
    in_features: int
    out_features: int

    @abstractmethod
    def forward(self, x: torch.Tensor) -> torch.Tensor: ...

    @abstractmethod
    def load_weight(self, weight: torch.Tensor, bias: torch.Tensor | None = None) -> None: ...

    @abstractmethod
    def weight_bytes(self) -> int: ...

    def swiglu(self, x: torch.Tensor, norm=None) -> torch.Tensor:
        """``silu(gate(x)) * up(x)`` for a layer whose rows are ``[gate; up]``:
        ``(T, K) -> (T, N / 2)``."""
        if norm is not None:
            raise ValueError(f"{type(self).__name__} takes no normed input")
        return kernels.silu_mul(self(x).reshape(-1, self.out_features), self.out_features // 2)

    def rope_append(self, x: torch.Tensor, positions, cos, sin, n_q_heads: int, n_kv_heads: int,
                    head_dim: int, slots, key_pool, value_pool, q_out=None, rows=None,
                    norm=None) -> torch.Tensor:
        """For a fused ``[q | k | v]`` layer: RoPE on q and k, k and v appended to the pools at
        ``slots``; returns q ``(T, n_q_heads, head_dim)``. ``rows``: ``kernels.rope_rows``."""
        if norm is not None:
            raise ValueError(f"{type(self).__name__} takes no normed input")
        qkv = self(x).reshape(-1, self.out_features)
        return kernels.rope_append(qkv, positions, cos, sin, n_q_heads, n_kv_heads, head_dim,
                                   slots, key_pool, value_pool, q_out=q_out)


class FP16Linear(LinearBase):
    """Dense layer (used for the fp16 lm_head and as the unquantised baseline)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.linear = nn.Linear(in_features, out_features, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.linear(x)

    def load_weight(self, weight: torch.Tensor, bias: torch.Tensor | None = None) -> None:
        if tuple(weight.shape) != (self.out_features, self.in_features):
            raise ValueError(
                f"weight shape {tuple(weight.shape)} does not match layer "
                f"({self.out_features}, {self.in_features})"
            )
        with torch.no_grad():
            self.linear.weight.copy_(weight)
            if bias is not None:
                if self.linear.bias is None:
                    raise ValueError("bias supplied to a layer constructed without one")
                self.linear.bias.copy_(bias)
            elif self.linear.bias is not None:
                raise ValueError("layer has a bias but none was supplied")

    def weight_bytes(self) -> int:
        total = self.linear.weight.numel() * self.linear.weight.element_size()
        if self.linear.bias is not None:
            total += self.linear.bias.numel() * self.linear.bias.element_size()
        return total


class QuantLinear(LinearBase):
    """Weight-only INT4/INT8 linear; quantises once in :meth:`load_weight`, on the HIP device."""

    packed: torch.Tensor
    scales: torch.Tensor
    bias: torch.Tensor | None

    def __init__(
        self,
        in_features: int,
        out_features: int,
        bias: bool = False,
        config: QuantConfig | None = None,
        device: torch.device | str | None = None,
    ) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.config = config or QuantConfig()
        if in_features % self.config.group_size:
            raise ValueError(
                f"in_features={in_features} is not divisible by group_size="
                f"{self.config.group_size}, so the final group would be ragged"
            )
        n_groups = in_features // self.config.group_size
        width = in_features // 2 if self.config.bits == 4 else in_features
        self.register_buffer(
            "packed", torch.zeros((out_features, width), dtype=torch.uint8, device=device)
        )
        self.register_buffer(
            "scales", torch.zeros((out_features, n_groups), dtype=torch.float16, device=device)
        )
        self.register_buffer(
            "bias",
            torch.zeros(out_features, dtype=torch.float16, device=device) if bias else None,
        )

    def _compute_device(self) -> torch.device:
        if self.packed.is_cuda:
            return self.packed.device
        if not torch.cuda.is_available():
            raise RuntimeError("QuantLinear quantises on the HIP device and none is available")
        return torch.device("cuda")

    def load_weight(self, weight: torch.Tensor, bias: torch.Tensor | None = None) -> None:
        if (bias is None) != (self.bias is None):
            raise ValueError(
                f"bias mismatch: layer was constructed with bias={self.bias is not None} but "
                f"load_weight was given bias={bias is not None}"
            )
        if tuple(weight.shape) != (self.out_features, self.in_features):
            raise ValueError(
                f"weight shape {tuple(weight.shape)} does not match layer "
                f"({self.out_features}, {self.in_features})"
            )
        dev = self._compute_device()
        packed, scales = quantize_packed(weight.detach().to(dev), self.config)
        with torch.no_grad():
            self.packed.copy_(packed)
            self.scales.copy_(scales)
            if bias is not None and self.bias is not None:
                self.bias.copy_(bias.detach().to(self.bias.device, torch.float16))

    def load_quantized(
        self, packed: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor | None = None
    ) -> None:
        """Take already-quantised buffers (e.g. a reference state dict) without re-quantising."""
        if tuple(packed.shape) != tuple(self.packed.shape) or packed.dtype != torch.uint8:
            raise ValueError(f"packed must be uint8 {tuple(self.packed.shape)}")
        if tuple(scales.shape) != tuple(self.scales.shape):
            raise ValueError(f"scales must be {tuple(self.scales.shape)}")
        if (bias is None) != (self.bias is None):
            raise ValueError("bias mismatch")
        with torch.no_grad():
            self.packed.copy_(packed)
            self.scales.copy_(scales.to(torch.float16))
            if bias is not None:
                self.bias.copy_(bias.to(torch.float16))

    def dequantized(self) -> torch.Tensor:
        return kernels.dequantize(
            self.packed, self.scales, self.in_features, self.config.bits, self.config.group_size
        )

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        return kernels.quant_linear(
            x, self.packed, self.scales, self.bias, self.in_features, self.out_features,
            self.config.bits, self.config.group_size, out=out,
        )

    def rope_append(self, x: torch.Tensor, positions, cos, sin, n_q_heads: int, n_kv_heads: int,
                    head_dim: int, slots, key_pool, value_pool, q_out=None, rows=None,
                    norm=None) -> torch.Tensor:
        """``LinearBase.rope_append`` in one launch for decode batches (``rows`` given);
        ``norm`` (``kernels.NormedInput``): x is a residual producer's ``xw``, normalised on the
        fly."""
        return kernels.quant_linear_rope_append(
            x, self.packed, self.scales, self.bias, self.in_features, self.config.bits,
            self.config.group_size, positions, cos, sin, n_q_heads, n_kv_heads, head_dim, slots,
            key_pool, value_pool, q_out=q_out, rows=rows, norm=norm,
        )

    def swiglu(self, x: torch.Tensor, norm=None) -> torch.Tensor:
        """``silu(gate(x)) * up(x)`` for a ``concat([gate, up])`` layer: ``(T, K) -> (T, N / 2)``,
        one launch for decode batches; ``norm`` as in ``rope_append``."""
        return kernels.quant_linear_swiglu(
            x, self.packed, self.scales, self.bias, self.in_features, self.out_features,
            self.config.bits, self.config.group_size, norm=norm,
        )

    def residual(self, x: torch.Tensor, hidden: torch.Tensor, partials: torch.Tensor,
                 next_norm_weight: torch.Tensor | None = None,
                 xw: torch.Tensor | None = None) -> int:
        """``hidden += self(x)`` in place plus what a normed input reads: the sums of squares and
        ``xw = fp16(next_norm_weight * hidden)`` (``kernels.quant_linear_residual``); returns the
        sums' count per token."""
        return kernels.quant_linear_residual(
            x, self.packed, self.scales, self.bias, self.in_features, self.out_features,
            self.config.bits, self.config.group_size, hidden, partials, next_norm_weight, xw,
        )

    def weight_bytes(self) -> int:
        total = (
            self.packed.numel() * self.packed.element_size()
            + self.scales.numel() * self.scales.element_size()
        )
        if self.bias is not None:
            total += self.bias.numel() * self.bias.element_size()
        return total

    @classmethod
    def concat(cls, layers: list[QuantLinear]) -> QuantLinear:
        """One layer computing ``cat([l(x) for l in layers], -1)`` in a single launch.

        Exact: every output row keeps its own codes and scales, so stacking rows (q/k/v, or
        gate/up) changes nothing but the launch count.
        """
        first = layers[0]
        for layer in layers:
            if layer.in_features != first.in_features or layer.config != first.config:
                raise ValueError("only layers with the same input size and config can be fused")
            if (layer.bias is None) != (first.bias is None):
                raise ValueError("either every fused layer has a bias or none does")
        fused = cls(
            first.in_features, sum(l.out_features for l in layers), bias=first.bias is not None,
            config=first.config, device=first.packed.device,
        )
        with torch.no_grad():
            fused.packed.copy_(torch.cat([l.packed for l in layers]))
            fused.scales.copy_(torch.cat([l.scales for l in layers]))
            if fused.bias is not None:
                fused.bias.copy_(torch.cat([l.bias for l in layers]))
        return fused


QUANTIZATION_SKIP_LIST: tuple[str, ...] = (
    "embed_tokens",
    "lm_head",
    "norm",
    "layernorm",
    "patch_embedding",
)


def should_quantize(module_name: str) -> bool:
    lowered = module_name.lower()
    return not any(skip in lowered for skip in QUANTIZATION_SKIP_LIST)
