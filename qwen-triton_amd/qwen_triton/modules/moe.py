"""Sparse MoE block (reference: qwen_triton/modules/moe.py:14-58).

Parameters keep the reference layout (``gate``, ``experts.{i}.{gate,up,down}_proj``,
optional ``shared_expert`` / ``shared_expert_gate``). The forward follows the
reference's routing semantics: fp32 softmax over router logits, top-k with ties
to the lower expert index, optional renormalisation, routing weights cast to the
activation dtype, per-expert SwiGLU on the tokens routed to it, scaled by the
routing weight and scatter-added in ascending expert order.

On the GPU the experts run as one sort/segment dispatch, grouped expert GEMMs
and an ordered combine (``kernels/moe_experts.py``) with the loop's rounding
points: without autograd through the inference kernels, with autograd through
``GroupedExperts``, whose backward gives the loop's gradients (input, routing
weights and every expert weight) from grouped products as well.
"""
from __future__ import annotations

import torch
from torch import nn

from qwen_triton import _native
from qwen_triton.configs import QwenTritonConfig
from qwen_triton.kernels.moe_experts import GroupedExperts, grouped_training_ok, moe_experts_forward
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
        self.moe_intermediate_size = config.moe_intermediate_size
        self._tables: tuple | None = None  # device pointer tables of the expert weights (not state)
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

    def _grouped_ok(self, flat: torch.Tensor, training: bool = False) -> bool:
        if torch.is_grad_enabled() != training or not flat.is_cuda or flat.dtype not in (torch.bfloat16, torch.float16):
            return False
        if training and not grouped_training_ok(flat.shape[1], self.moe_intermediate_size):
            return False
        if flat.shape[1] % 8 or self.moe_intermediate_size % 8 or not _native.available():
            return False
        ws = [(e.gate_proj.weight, e.up_proj.weight, e.down_proj.weight) for e in self.experts]
        g0, d0 = ws[0][0], ws[0][2]
        return all(
            e.gate_proj.bias is None and e.up_proj.bias is None and e.down_proj.bias is None for e in self.experts
        ) and all(
            g.dtype == flat.dtype and u.dtype == flat.dtype and d.dtype == flat.dtype and g.is_cuda
            and g.stride() == g0.stride() and u.stride() == g0.stride() and d.stride() == d0.stride()
            and g.stride(1) == 1 and d.stride(1) == 1 and g.stride(0) % 8 == 0 and d.stride(0) % 8 == 0
            and g.data_ptr() % 16 == 0 and u.data_ptr() % 16 == 0 and d.data_ptr() % 16 == 0
            for g, u, d in ws)

    def _expert_tables(self, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
        ptrs = [(e.gate_proj.weight.data_ptr(), e.up_proj.weight.data_ptr(), e.down_proj.weight.data_ptr())
                for e in self.experts]
        key = (device, tuple(ptrs))
        if self._tables is None or self._tables[0] != key:
            gu = torch.tensor([p for g, u, _ in ptrs for p in (g, u)], dtype=torch.int64, device=device)
            dn = torch.tensor([d for _, _, d in ptrs], dtype=torch.int64, device=device)
            self._tables = (key, gu, dn)
        return self._tables[1], self._tables[2]

    def experts_forward(self, flat: torch.Tensor, routing_weights: torch.Tensor, selected: torch.Tensor) -> torch.Tensor:
        strides = (self.experts[0].gate_proj.weight.stride(0), self.experts[0].down_proj.weight.stride(0))
        if self._grouped_ok(flat):
            gu, dn = self._expert_tables(flat.device)
            return moe_experts_forward(flat, routing_weights, selected, gu, dn, self.num_experts,
                                       self.moe_intermediate_size, strides)
        if self._grouped_ok(flat, training=True):
            gu, dn = self._expert_tables(flat.device)
            weights = [p for e in self.experts for p in (e.gate_proj.weight, e.up_proj.weight, e.down_proj.weight)]
            return GroupedExperts.apply(flat, routing_weights, selected, gu, dn, self.num_experts,
                                        self.moe_intermediate_size, strides[0], strides[1], *weights)
        out = torch.zeros_like(flat)
        expert_mask = triton_one_hot(selected, self.num_experts).permute(2, 1, 0)
        hit = torch.nonzero(expert_mask.sum(dim=(-1, -2)) > 0, as_tuple=False).view(-1)
        for e in hit.tolist():
            slot, tok = torch.where(expert_mask[e])
            cur = self.experts[e](flat[tok]) * routing_weights[tok, slot, None]
            out = triton_index_add(out, cur.to(flat.dtype), tok)
        return out
