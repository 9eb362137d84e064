"""Qwen3-Next / Qwen3.5 gated-delta linear attention block.

Reference: qwen_triton/modules/linear_attention.py:23-155 (``Qwen3NextLinearAttention``), with the
parameter names of the HF checkpoints: ``in_proj_qkvz``, ``in_proj_ba``, ``conv1d`` (depthwise,
no bias), ``dt_bias``, ``A_log``, ``norm`` (gated RMSNorm) and ``out_proj``.

Per token: the projections give q, k, v, the output gate z and the per-head b, a; q, k and v go
through a causal depthwise convolution over time with SiLU (its last ``kernel - 1`` raw inputs are
the cache's conv state); beta = sigmoid(b), the log-decay g = -exp(A_log) * softplus(a + dt_bias);
q and k are repeated to the value heads and L2-normalised, and the gated delta rule
(``gated_delta_rule_sequence``, one HIP launch for the whole sequence) gives the outputs and the
new recurrent state; the output is RMSNorm-ed per head, gated by SiLU(z) and projected back.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from qwen_triton.configs import QwenTritonConfig
from qwen_triton.kernels import gated_delta_rule_sequence
from qwen_triton.modules.linear import TritonLinear
from qwen_triton.modules.norms import QwenRMSNormGated


def _masked(hidden_states: torch.Tensor, attention_mask: torch.Tensor | None) -> torch.Tensor:
    """Zero padded positions (a [B, S] mask of a padded multi-sequence batch), as the reference does."""
    if attention_mask is not None and attention_mask.dim() == 2 and attention_mask.shape[0] > 1 \
            and attention_mask.shape[1] > 1:
        return hidden_states * attention_mask[:, :, None].to(hidden_states.dtype)
    return hidden_states


def _l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).sum(dim=-1, keepdim=True) + eps)


class Qwen3NextLinearAttention(nn.Module):
    def __init__(self, config: QwenTritonConfig, layer_idx: int) -> None:
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.hidden_size = config.hidden_size
        self.num_k_heads = config.linear_num_key_heads
        self.num_v_heads = config.linear_num_value_heads
        self.head_k_dim = config.linear_key_head_dim
        self.head_v_dim = config.linear_value_head_dim
        if self.num_k_heads <= 0 or self.num_v_heads % self.num_k_heads:
            raise ValueError("linear attention needs value heads that are a multiple of the key heads")
        self.key_dim = self.num_k_heads * self.head_k_dim
        self.value_dim = self.num_v_heads * self.head_v_dim
        self.conv_kernel_size = config.linear_conv_kernel_dim
        self.conv_dim = 2 * self.key_dim + self.value_dim
        self.conv1d = nn.Conv1d(self.conv_dim, self.conv_dim, kernel_size=self.conv_kernel_size,
                                groups=self.conv_dim, bias=False, padding=0)
        self.in_proj_qkvz = TritonLinear(self.hidden_size, 2 * self.key_dim + 2 * self.value_dim, bias=False)
        self.in_proj_ba = TritonLinear(self.hidden_size, 2 * self.num_v_heads, bias=False)
        self.dt_bias = nn.Parameter(torch.ones(self.num_v_heads))
        self.A_log = nn.Parameter(torch.empty(self.num_v_heads).uniform_(0, 16).log_())
        self.norm = QwenRMSNormGated(self.head_v_dim, eps=config.rms_norm_eps)
        self.out_proj = TritonLinear(self.value_dim, self.hidden_size, bias=False)

    def _split(self, qkvz: torch.Tensor, ba: torch.Tensor):
        """The checkpoint layout groups the projections per key head: [q | k | v | z] of one key
        head (v and z covering its nv/nk value heads), then [b | a] the same way."""
        B, S = qkvz.shape[:2]
        r = self.num_v_heads // self.num_k_heads
        g = qkvz.view(B, S, self.num_k_heads, 2 * self.head_k_dim + 2 * r * self.head_v_dim)
        q, k, v, z = torch.split(g, [self.head_k_dim, self.head_k_dim, r * self.head_v_dim, r * self.head_v_dim],
                                 dim=3)
        b, a = torch.split(ba.view(B, S, self.num_k_heads, 2 * r), [r, r], dim=3)
        return (q, k, v.reshape(B, S, self.num_v_heads, self.head_v_dim),
                z.reshape(B, S, self.num_v_heads, self.head_v_dim), b.reshape(B, S, self.num_v_heads),
                a.reshape(B, S, self.num_v_heads))

    def _conv(self, mixed: torch.Tensor, cache_params) -> torch.Tensor:
        """Causal depthwise convolution over time + SiLU of mixed [B, C, S]; the conv state carries
        the previous chunk's last kernel - 1 raw inputs."""
        seq = mixed.shape[-1]
        prev = None if cache_params is None else cache_params.conv_states[self.layer_idx]
        if prev is None:
            prev = mixed.new_zeros(mixed.shape[0], mixed.shape[1], self.conv_kernel_size - 1)
        full = torch.cat((prev.to(mixed.dtype), mixed), dim=-1)
        if cache_params is not None:
            cache_params.conv_states[self.layer_idx] = full[:, :, full.shape[-1] - (self.conv_kernel_size - 1):]
        out = F.conv1d(full, self.conv1d.weight, None, groups=self.conv_dim)
        return F.silu(out[:, :, -seq:])

    def forward(self, hidden_states: torch.Tensor, cache_params=None, cache_position: torch.LongTensor | None = None,
                attention_mask: torch.Tensor | None = None) -> torch.Tensor:
        del cache_position
        x = _masked(hidden_states, attention_mask)
        B, S, _ = x.shape
        q, k, v, z, b, a = self._split(self.in_proj_qkvz(x), self.in_proj_ba(x))
        mixed = torch.cat((q.reshape(B, S, -1), k.reshape(B, S, -1), v.reshape(B, S, -1)), dim=-1)
        mixed = self._conv(mixed.transpose(1, 2), cache_params).transpose(1, 2)
        q, k, v = torch.split(mixed, [self.key_dim, self.key_dim, self.value_dim], dim=-1)
        q = q.reshape(B, S, self.num_k_heads, self.head_k_dim)
        k = k.reshape(B, S, self.num_k_heads, self.head_k_dim)
        v = v.reshape(B, S, self.num_v_heads, self.head_v_dim)
        beta = b.sigmoid()
        g = -self.A_log.float().exp() * F.softplus(a.float() + self.dt_bias)
        r = self.num_v_heads // self.num_k_heads
        if r > 1:
            q = q.repeat_interleave(r, dim=2)
            k = k.repeat_interleave(r, dim=2)
        state = None if cache_params is None else cache_params.recurrent_states[self.layer_idx]
        out, state = gated_delta_rule_sequence(_l2norm(q), _l2norm(k), v, g, beta, initial_state=state)
        if cache_params is not None:
            cache_params.recurrent_states[self.layer_idx] = state
        out = self.norm(out.reshape(-1, self.head_v_dim), z.reshape(-1, self.head_v_dim))
        return self.out_proj(out.reshape(B, S, self.value_dim))
