"""Qwen3-Next gated-delta linear attention block.

Reference: qwen_triton/modules/linear_attention.py:23-155. The Qwen3-Next /
Qwen3.5 family is outside this library's scope; the class is kept so imports
resolve, and constructing it explains that.
"""
from __future__ import annotations

from torch import nn


class Qwen3NextLinearAttention(nn.Module):
    def __init__(self, config, layer_idx: int) -> None:
        super().__init__()
        raise NotImplementedError(
            "Qwen3-Next/Qwen3.5 linear-attention layers are not supported by the MI355X operator stack"
        )
