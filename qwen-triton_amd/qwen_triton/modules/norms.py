"""RMSNorm modules (reference: qwen_triton/modules/norms.py:9-36)."""
from __future__ import annotations

import torch
from torch import nn

from qwen_triton.kernels import rmsnorm, silu_mul


class QwenRMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-6, one_plus_weight: bool = False) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.full((hidden_size,), 0.0 if one_plus_weight else 1.0))
        self.eps = eps
        self.one_plus_weight = one_plus_weight

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return rmsnorm(hidden_states, self.weight, eps=self.eps, one_plus_weight=self.one_plus_weight)

    def extra_repr(self) -> str:
        return f"{tuple(self.weight.shape)}, eps={self.eps}, one_plus_weight={self.one_plus_weight}"


class QwenRMSNormGated(nn.Module):
    """RMSNorm of the linear-attention output gated by SiLU(gate) (Qwen3-Next / Qwen3.5):
    silu(gate) * rmsnorm(x) * weight, the norm in fp32 with one rounding (the RMSNorm kernel), then
    the SiLU-mul kernel (reference: qwen_triton/modules/norms.py:24-36)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, hidden_states: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        normed = rmsnorm(hidden_states, self.weight, eps=self.eps)
        return silu_mul(gate.to(normed.dtype), normed)
