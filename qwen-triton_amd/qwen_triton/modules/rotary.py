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
        # (device, dtype) -> [P, 2 * rotary_dim] table, row p = cos(p) | sin(p); not module state
        self._tables: dict[tuple, torch.Tensor] = {}

    def _apply(self, fn, recurse=True):
        # Module dtype casts (model.to(torch.bfloat16)) must not round the frequencies: a bf16
        # inv_freq moves the RoPE angle at position 2048 by up to ~4 radians. Device moves apply.
        inv = self.inv_freq
        super()._apply(fn, recurse)
        self.inv_freq = inv.to(device=self.inv_freq.device, dtype=torch.float32)
        self._tables = {}
        return self

    def _cos_sin(self, position_ids: torch.Tensor, device, dtype) -> tuple[torch.Tensor, torch.Tensor]:
        inv = self.inv_freq.to(device=device, dtype=torch.float32)
        freqs = position_ids.to(torch.float32)[:, :, None] * inv[None, None, :]
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(dtype), emb.sin().to(dtype)

    def table(self, device, dtype, positions: int) -> torch.Tensor:
        """Rows cos(p) | sin(p) for p < P (P a power of two, at least ``positions``), computed once
        by the same elementwise ops as the per-call path, so every row equals what that path gives
        for position p bit for bit."""
        key = (torch.device(device), dtype)
        t = self._tables.get(key)
        if t is None or t.shape[0] < positions:
            rows = max(256, 1 << (max(positions, 1) - 1).bit_length())
            cos, sin = self._cos_sin(torch.arange(rows, device=device)[None], device, dtype)
            t = torch.cat((cos[0], sin[0]), dim=-1).contiguous()
            self._tables[key] = t
        return t

    @torch.no_grad()
    def forward(self, hidden_states: torch.Tensor, position_ids: torch.Tensor,
                max_position: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """cos/sin of shape [position_ids.shape[0], S, rotary_dim] in the activation dtype.

        With ``max_position`` (a bound on every position id, known to the caller) the rows are
        gathered from the cached table in one launch instead of being computed per call (which
        takes seven elementwise launches); they are views of one gathered [B, S, 2 * rot] tensor."""
        if max_position is None or not hidden_states.is_cuda:
            return self._cos_sin(position_ids, hidden_states.device, hidden_states.dtype)
        rot = self.inv_freq.shape[0] * 2
        t = self.table(hidden_states.device, hidden_states.dtype, max_position + 1)
        rows = torch.nn.functional.embedding(position_ids, t)
        return rows[..., :rot], rows[..., rot:]


def apply_rotary_pos_emb(query, key, cos, sin):
    return apply_rope(query, key, cos, sin)
