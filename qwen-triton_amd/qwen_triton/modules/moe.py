"""Sparse MoE block (reference: qwen_triton/modules/moe.py:14-58).

Parameters keep the reference layout (``gate``, ``experts.{i}.{gate,up,down}_proj``,
optional ``shared_expert`` / ``shared_expert_gate``). The forward follows the
reference's routing semantics: fp32 softmax over router logits, top-k with ties
to the lower expert index, optional renormalisation, routing weights cast to the
activation dtype, per-expert SwiGLU on the tokens routed to it, scaled by the
routing weight and scatter-added in ascending expert order.
"""
from __future__ import annotations

import torch
from torch import nn

from qwen_triton.configs import QwenTritonConfig
from qwen_triton.kernels.moe_routing import triton_index_add, triton_one_hot, triton_topk
from qwen_triton.kernels.sigmoid_mul import sigmoid_mul
from qwen_triton.kernels.softmax import triton_softmax
from qwen_triton.modules.linear import TritonLinear
from qwen_triton.modules.mlp import QwenMLP


class QwenSparseMoeBlock(nn.Module):
    def __init__(self, config: QwenTritonConfig) -> None:
        super().__init__()
        self.hidden_size = config.hidden_size
        self.num_experts = config.num_experts
        self.top_k = config.num_experts_per_tok
        self.norm_topk_prob = config.norm_topk_prob
        self.gate = TritonLinear(config.hidden_size, config.num_experts, bias=False)
        self.experts = nn.ModuleList(
            [QwenMLP(config.hidden_size, config.moe_intermediate_size) for _ in range(config.num_experts)]
        )
        self.shared_expert = None
        self.shared_expert_gate = None
        if config.shared_expert_intermediate_size > 0:
            self.shared_expert = QwenMLP(config.hidden_size, config.shared_expert_intermediate_size)
            self.shared_expert_gate = TritonLinear(config.hidden_size, 1, bias=False)

    def route(self, router_logits: torch.Tensor, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
        weights = triton_softmax(router_logits.float())
        weights, selected = triton_topk(weights, self.top_k)
        if self.norm_topk_prob:
            weights = weights / weights.sum(dim=-1, keepdim=True)
        return weights.to(dtype), selected

    def forward(self, hidden_states: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        batch, seq, hidden = hidden_states.shape
        flat = hidden_states.view(-1, hidden)
        router_logits = self.gate(flat)
        routing_weights, selected = self.route(router_logits, flat.dtype)
        out = self.experts_forward(flat, routing_weights, selected)
        if self.shared_expert is not None and self.shared_expert_gate is not None:
            shared = self.shared_expert(flat)
            gate_value = self.shared_expert_gate(flat)
            out = out + sigmoid_mul(shared, gate_value.expand_as(shared))
        return out.view(batch, seq, hidden), router_logits

    def experts_forward(self, flat: torch.Tensor, routing_weights: torch.Tensor, selected: torch.Tensor) -> torch.Tensor:
        out = torch.zeros_like(flat)
        expert_mask = triton_one_hot(selected, self.num_experts).permute(2, 1, 0)
        hit = torch.nonzero(expert_mask.sum(dim=(-1, -2)) > 0, as_tuple=False).view(-1)
        for e in hit.tolist():
            slot, tok = torch.where(expert_mask[e])
            cur = self.experts[e](flat[tok]) * routing_weights[tok, slot, None]
            out = triton_index_add(out, cur.to(flat.dtype), tok)
        return out
