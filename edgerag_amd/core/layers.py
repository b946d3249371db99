"""Parameters and tables of a decoder layer's elementwise ops, on packed token-major tensors.

* :class:`RMSNorm` holds the norm weight; its ``forward`` runs ``edgerag_rmsnorm`` (fp32 variance,
  ``x * rsqrt(var + eps)`` in fp32, cast to the input dtype *before* the weight multiply, as
  ``edgerag/core/layers.py:40-47``).
* :class:`RotaryTable` holds cos/sin for every logical position: ``inv_freq = 1 / theta^(2i/d)``
  in fp32, ``freqs = pos * inv_freq``, ``emb = cat(freqs, freqs)``, cos/sin in fp32 cast to the
  activation dtype (``layers.py:64-90``). The products ``pos * inv_freq`` are single fp32
  multiplies, so a table indexed by position holds exactly the values the reference recomputes per
  step. The decoder's RoPE (halves convention, ``layers.py:93-114``) runs in the HIP kernels that
  read these tables.
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
        """RMSNorm over the last axis, on the device (``edgerag_rmsnorm``)."""
        from edgerag_amd import kernels

        flat = x.reshape(-1, x.shape[-1])
        return kernels.rmsnorm(flat.contiguous(), self.weight, self.eps).view(x.shape)


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
