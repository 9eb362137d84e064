"""SwiGLU MLP (reference: qwen_triton/modules/mlp.py:10-22).

Inference with up to 128 tokens computes gate, up and silu(gate) * up in one
grouped launch with the arithmetic of the separate kernels.
"""
from __future__ import annotations

import torch
from torch import nn

from qwen_triton.kernels import silu_mul
from qwen_triton.kernels.matmul import linear_group, linear_group_ok
from qwen_triton.modules.linear import TritonLinear


class QwenMLP(nn.Module):
    def __init__(self, hidden_size: int, intermediate_size: int) -> None:
        super().__init__()
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.gate_proj = TritonLinear(hidden_size, intermediate_size, bias=False)
        self.up_proj = TritonLinear(hidden_size, intermediate_size, bias=False)
        self.down_proj = TritonLinear(intermediate_size, hidden_size, bias=False)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        gate_up = [self.gate_proj.weight, self.up_proj.weight]
        if (not torch.is_grad_enabled() and self.gate_proj.bias is None and self.up_proj.bias is None
                and linear_group_ok(hidden_states, gate_up)):
            return self.down_proj(linear_group(hidden_states, gate_up, gated=True))
        return self.down_proj(silu_mul(self.gate_proj(hidden_states), self.up_proj(hidden_states)))
