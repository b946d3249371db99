"""Decoder-layer ops around the hot path, on packed token-major tensors ``(T, ...)``.

The arithmetic follows the reference layer by layer (``edgerag/core/layers.py``):

* :class:`RMSNorm` -- fp32 variance, ``x * rsqrt(var + eps)`` in fp32, cast back to the input
  dtype *before* the weight multiply (``layers.py:40-47``);
* :class:`RotaryTable` -- ``inv_freq = 1 / theta^(2i/d)`` in fp32, ``freqs = pos * inv_freq``,
  ``emb = cat(freqs, freqs)``, cos/sin in fp32 cast to the activation dtype (``layers.py:64-90``);
  positions are *logical* (P-03). The products ``pos * inv_freq`` are single fp32 multiplies, so a
  table indexed by position holds exactly the values the reference recomputes per step;
* :func:`apply_rope` -- the halves convention ``x * cos + rotate_half(x) * sin`` with
  ``rotate_half(x) = [-x2, x1]`` (``layers.py:93-114``);
* :func:`silu_mul` -- ``silu(gate) * up`` of SwiGLU (``layers.py:341``).

The decoder's forward runs the fused HIP kernels (``edgerag_rmsnorm`` with the residual add,
``edgerag_rope_append``, ``edgerag_silu_mul``); the modules here hold the parameters and tables
those kernels read, and their ``forward`` methods state the same arithmetic in PyTorch.
"""

from __future__ import annotations

import torch
from torch import nn


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float, device=None, dtype=torch.float16) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype),
                                   requires_grad=False)
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        input_dtype = x.dtype
        xf = x.to(torch.float32)
        variance = xf.pow(2).mean(-1, keepdim=True)
        xf = xf * torch.rsqrt(variance + self.eps)
        return self.weight * xf.to(input_dtype)


class RotaryTable(nn.Module):
    """cos/sin for every logical position below ``max_positions``, in the activation dtype."""

    def __init__(self, head_dim: int, theta: float, max_positions: int, device=None,
                 dtype=torch.float16) -> None:
        super().__init__()
        inv_freq = 1.0 / (
            theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim)
        )
        pos = torch.arange(max_positions, dtype=torch.float32)
        freqs = pos[:, None] * inv_freq[None, :]
        emb = torch.cat((freqs, freqs), dim=-1)
        self.register_buffer("cos", emb.cos().to(dtype).to(device), persistent=False)
        self.register_buffer("sin", emb.sin().to(dtype).to(device), persistent=False)

    def forward(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        return self.cos[positions], self.sin[positions]


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``x (T, H, d)``, ``cos``/``sin`` ``(T, d)`` broadcast over heads."""
    return x * cos[:, None, :] + rotate_half(x) * sin[:, None, :]


def silu_mul(gate_up: torch.Tensor, intermediate: int) -> torch.Tensor:
    """``silu(gate) * up`` for the fused ``[gate | up]`` projection output ``(T, 2 I)``."""
    return nn.functional.silu(gate_up[:, :intermediate]) * gate_up[:, intermediate:]
