"""Gated delta rule recurrence (Qwen3-Next / Qwen3.5 linear attention) on the HIP library.

Reference: qwen_triton/kernels/linear_attention.py:35-189 (torch step :35-51, Triton step kernel
:54-101, launcher :104-127, sequence driver :130-189). The reference launches its step kernel once
per token from a Python loop; here one launch (``qh_gated_delta_rule``) runs the whole sequence
with each (sequence, head) state held in registers. Same signature and results: outputs in the
value dtype, the final state in fp32, the query scaled by key_dim ** -0.5 in its own dtype.

The kernel has no backward (neither has the reference's Triton path, whose outputs leave
autograd): when a gradient is required the differentiable torch recurrence runs instead.
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, Unsupported, needs_grad

_GUARD = OpGuard("LinearAttention")


def _torch_gated_delta_rule_step(state, query, key, value, decay, beta):
    state = state * decay.exp()[:, None, None]
    kv_mem = torch.einsum("nkv,nk->nv", state, key)
    delta = (value - kv_mem) * beta[:, None]
    state = state + key[:, :, None] * delta[:, None, :]
    out = torch.einsum("nkv,nk->nv", state, query)
    return out, state


def _torch_sequence(query, key, value, decay, beta, initial_state):
    B, S, H, K = query.shape
    Vd = value.shape[-1]
    query = query * (K ** -0.5)
    if initial_state is None:
        state = torch.zeros((B * H, K, Vd), device=query.device, dtype=torch.float32)
    else:
        state = initial_state.reshape(B * H, K, Vd).to(torch.float32)
    outs = []
    for t in range(S):
        out_t, state = _torch_gated_delta_rule_step(
            state,
            query[:, t].reshape(B * H, K).float(),
            key[:, t].reshape(B * H, K).float(),
            value[:, t].reshape(B * H, Vd).float(),
            decay[:, t].reshape(B * H).float(),
            beta[:, t].reshape(B * H).float(),
        )
        outs.append(out_t.view(B, H, Vd))
    outputs = torch.stack(outs, dim=1) if outs else value.new_zeros((B, 0, H, Vd), dtype=torch.float32)
    return outputs.to(value.dtype), state.view(B, H, K, Vd)


def _native_sequence(query, key, value, decay, beta, initial_state):
    _native.require_device(query, key, value, decay, beta)
    if query.dim() != 4 or key.shape != query.shape or value.dim() != 4 or value.shape[:3] != query.shape[:3]:
        raise Unsupported(f"gated delta rule expects q/k [B,S,H,K] and v [B,S,H,V]; got {tuple(query.shape)}, "
                          f"{tuple(key.shape)}, {tuple(value.shape)}")
    if not (query.dtype == key.dtype == value.dtype) or query.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise Unsupported("gated delta rule kernel takes q/k/v of one float dtype")
    B, S, H, K = query.shape
    Vd = value.shape[-1]
    if K > 128:
        raise Unsupported(f"gated delta rule kernel takes key head dims up to 128, got {K}")
    if query.stride(-1) != 1 or key.stride() != query.stride():
        query, key = query.contiguous(), key.contiguous()
    if value.stride(-1) != 1:
        value = value.contiguous()
    g = decay.to(torch.float32).expand(B, S, H).contiguous()
    bt = beta.to(torch.float32).expand(B, S, H).contiguous()
    state_in = None
    if initial_state is not None:
        state_in = initial_state.reshape(B, H, K, Vd).to(torch.float32).contiguous()
    out = torch.empty((B, S, H, Vd), dtype=value.dtype, device=value.device)
    state = torch.empty((B, H, K, Vd), dtype=torch.float32, device=value.device)
    _native.call("qh_gated_delta_rule", query.data_ptr(), key.data_ptr(), query.stride(0), query.stride(1),
                 query.stride(2), value.data_ptr(), value.stride(0), value.stride(1), value.stride(2), g.data_ptr(),
                 bt.data_ptr(), g.stride(0), g.stride(1), g.stride(2),
                 None if state_in is None else state_in.data_ptr(), state.data_ptr(), out.data_ptr(), out.stride(0),
                 out.stride(1), out.stride(2), B, S, H, K, Vd, float(K ** -0.5), _native.dtype_code(value.dtype),
                 _native.stream(value.device))
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
    """query/key [B,S,H,K], value [B,S,H,V], decay/beta [B,S,H] -> ([B,S,H,V], [B,H,K,V] fp32)."""
    if not _GUARD.use_native(use_triton, query, key, value) or needs_grad(query, key, value, decay, beta,
                                                                           initial_state):
        return _torch_sequence(query, key, value, decay, beta, initial_state)
    try:
        return _native_sequence(query, key, value, decay, beta, initial_state)
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_sequence(query, key, value, decay, beta, initial_state)
