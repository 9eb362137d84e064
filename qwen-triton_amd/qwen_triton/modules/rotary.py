"""Rotary embedding tables and application (reference: qwen_triton/modules/rotary.py:10-35)."""
from __future__ import annotations

import torch
from torch import nn

from qwen_triton.configs import QwenTritonConfig
from qwen_triton.kernels import apply_rope


class QwenRotaryEmbedding(nn.Module):
    def __init__(self, config: QwenTritonConfig) -> None:
        super().__init__()
        self.config = config
        dim = config.rotary_dim
        inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
        self.register_buffer("inv_freq", inv_freq, persistent=False)

    def _apply(self, fn, recurse=True):
        # Module dtype casts (model.to(torch.bfloat16)) must not round the frequencies: a bf16
        # inv_freq moves the RoPE angle at position 2048 by up to ~4 radians. Device moves apply.
        inv = self.inv_freq
        super()._apply(fn, recurse)
        self.inv_freq = inv.to(device=self.inv_freq.device, dtype=torch.float32)
        return self

    @torch.no_grad()
    def forward(self, hidden_states: torch.Tensor, position_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """cos/sin of shape [position_ids.shape[0], S, rotary_dim] in the activation dtype."""
        inv = self.inv_freq.to(device=hidden_states.device, dtype=torch.float32)
        freqs = position_ids.to(torch.float32)[:, :, None] * inv[None, None, :]
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(hidden_states.dtype), emb.sin().to(hidden_states.dtype)


def apply_rotary_pos_emb(query, key, cos, sin):
    return apply_rope(query, key, cos, sin)
