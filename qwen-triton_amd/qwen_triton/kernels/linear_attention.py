"""Gated delta rule recurrence (Qwen3-Next / Qwen3.5 linear attention).

Reference: qwen_triton/kernels/linear_attention.py:35-189. This family is out of
scope for the MI355X operator library (no Qwen3-Next configuration is
benchmarked), so only the torch recurrence is provided, with the reference's
signature, so that imports and callers keep working.
"""
from __future__ import annotations

import torch


def _torch_gated_delta_rule_step(state, query, key, value, decay, beta):
    state = state * decay.exp()[:, None, None]
    kv_mem = torch.einsum("nkv,nk->nv", state, key)
    delta = (value - kv_mem) * beta[:, None]
    state = state + key[:, :, None] * delta[:, None, :]
    out = torch.einsum("nkv,nk->nv", state, query)
    return out, state


def gated_delta_rule_sequence(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    decay: torch.Tensor,
    beta: torch.Tensor,
    initial_state: torch.Tensor | None = None,
    use_triton: bool | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """query/key [B,S,H,K], value [B,S,H,V], decay/beta [B,S,H] -> ([B,S,H,V], [B,H,K,V])."""
    del use_triton
    B, S, H, K = query.shape
    Vd = value.shape[-1]
    query = query * (K ** -0.5)
    if initial_state is None:
        state = torch.zeros((B * H, K, Vd), device=query.device, dtype=torch.float32)
    else:
        state = initial_state.reshape(B * H, K, Vd).to(torch.float32)
    outputs = torch.empty((B, S, H, Vd), device=value.device, dtype=torch.float32)
    for t in range(S):
        out_t, state = _torch_gated_delta_rule_step(
            state,
            query[:, t].reshape(B * H, K).float(),
            key[:, t].reshape(B * H, K).float(),
            value[:, t].reshape(B * H, Vd).float(),
            decay[:, t].reshape(B * H).float(),
            beta[:, t].reshape(B * H).float(),
        )
        outputs[:, t] = out_t.view(B, H, Vd)
    return outputs.to(value.dtype), state.view(B, H, K, Vd)
