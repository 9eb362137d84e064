"""RMSNorm ``x * rsqrt(mean(x^2) + eps) * (w or 1 + w)`` on the HIP library.

Reference: qwen_triton/kernels/rmsnorm.py:35-271 (torch fallbacks :35-62,
forward kernel :101-133, backward kernel :148-196, autograd :199-247, public op
:250-271). The backward's weight gradient is a deterministic two-stage column
sum instead of the reference's per-element fp32 atomics (:196).
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, needs_grad, Unsupported

_GUARD = OpGuard("RMSNorm")


def _torch_rmsnorm(hidden_states: torch.Tensor, weight: torch.Tensor, eps: float, one_plus_weight: bool) -> torch.Tensor:
    input_dtype = hidden_states.dtype
    x = hidden_states.to(torch.float32)
    variance = x.pow(2).mean(dim=-1, keepdim=True)
    scale = 1.0 + weight.to(torch.float32) if one_plus_weight else weight.to(torch.float32)
    return (x * torch.rsqrt(variance + eps) * scale).to(input_dtype)


def _torch_rmsnorm_backward(hidden_states, weight, grad_output, eps, one_plus_weight):
    x = hidden_states.to(torch.float32)
    g = grad_output.to(torch.float32)
    scale = 1.0 + weight.to(torch.float32) if one_plus_weight else weight.to(torch.float32)
    inv = torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)
    grad_weight = (g * x * inv).sum(dim=tuple(range(g.ndim - 1)))
    dot = (g * scale * x).sum(dim=-1, keepdim=True)
    grad_x = g * scale * inv - x * (inv.pow(3) / x.shape[-1]) * dot
    return grad_x.to(hidden_states.dtype), grad_weight.to(weight.dtype)


def _native_rmsnorm(hidden_states: torch.Tensor, weight: torch.Tensor, eps: float, one_plus_weight: bool) -> torch.Tensor:
    _native.require_device(hidden_states, weight)
    cols = hidden_states.shape[-1]
    if weight.numel() != cols:
        raise Unsupported(f"rmsnorm weight has {weight.numel()} elements, expected {cols}")
    x = hidden_states.contiguous()
    w = weight.contiguous()
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    rows = x.numel() // cols if cols else 0
    _native.call("qh_rmsnorm_fwd", x.data_ptr(), w.data_ptr(), out.data_ptr(), rows, cols, float(eps),
                 int(bool(one_plus_weight)), _native.dtype_code(x.dtype), _native.dtype_code(w.dtype),
                 _native.stream(x.device))
    return out


def _native_rmsnorm_backward(hidden_states, weight, grad_output, eps, one_plus_weight):
    x = hidden_states.contiguous()
    w = weight.contiguous()
    g = grad_output.contiguous().to(x.dtype)
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    dt = _native.dtype_code(x.dtype)
    gx = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    gw = torch.empty(w.shape, dtype=w.dtype, device=w.device)
    nbytes = _native.call("qh_rmsnorm_bwd_workspace", rows, cols, dt)
    ws = _native.workspace(nbytes, x.device)
    _native.call("qh_rmsnorm_bwd", x.data_ptr(), w.data_ptr(), g.data_ptr(), gx.data_ptr(), gw.data_ptr(),
                 ws.data_ptr(), ws.numel(), rows, cols, float(eps), int(bool(one_plus_weight)), dt,
                 _native.dtype_code(w.dtype), _native.stream(x.device))
    return gx.view_as(hidden_states), gw


class _RMSNormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden_states, weight, eps, one_plus_weight):
        ctx.eps = eps
        ctx.one_plus_weight = one_plus_weight
        ctx.save_for_backward(hidden_states, weight)
        return _native_rmsnorm(hidden_states, weight, eps, one_plus_weight)

    @staticmethod
    def backward(ctx, grad_output):
        hidden_states, weight = ctx.saved_tensors
        try:
            gx, gw = _native_rmsnorm_backward(hidden_states, weight, grad_output, ctx.eps, ctx.one_plus_weight)
        except Exception as exc:
            _GUARD.failed(exc, "backward kernel")
            gx, gw = _torch_rmsnorm_backward(hidden_states, weight, grad_output, ctx.eps, ctx.one_plus_weight)
        return gx, gw, None, None


def rmsnorm(
    hidden_states: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
    one_plus_weight: bool = False,
    use_triton: bool | None = None,
) -> torch.Tensor:
    if not _GUARD.use_native(use_triton, hidden_states, weight):
        return _torch_rmsnorm(hidden_states, weight, eps, one_plus_weight)
    try:
        if needs_grad(hidden_states, weight):
            return _RMSNormFunction.apply(hidden_states, weight, eps, one_plus_weight)
        return _native_rmsnorm(hidden_states, weight, eps, one_plus_weight)
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_rmsnorm(hidden_states, weight, eps, one_plus_weight)


def add_rmsnorm_ok(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor) -> bool:
    """True when the fused residual-add + RMSNorm pass applies (inference on GPU)."""
    return (not torch.is_grad_enabled() and x.is_cuda and x.dtype in (torch.bfloat16, torch.float16)
            and residual.shape == x.shape and residual.dtype == x.dtype and x.is_contiguous()
            and residual.is_contiguous() and weight.is_contiguous() and weight.dim() == 1
            and weight.shape[0] == x.shape[-1] and weight.dtype in (torch.float32, torch.float16, torch.bfloat16)
            and _native.available())


def add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                one_plus_weight: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """``s = x + residual`` and ``rmsnorm(s)`` in one pass (no autograd); equals
    ``residual_add`` followed by ``rmsnorm`` exactly. Returns ``(s, rmsnorm(s))``."""
    cols = x.shape[-1]
    s = torch.empty_like(x)
    y = torch.empty_like(x)
    _native.call("qh_add_rmsnorm", x.data_ptr(), residual.data_ptr(), weight.data_ptr(), s.data_ptr(), y.data_ptr(),
                 x.numel() // max(cols, 1), cols, float(eps), int(one_plus_weight), _native.dtype_code(x.dtype),
                 _native.dtype_code(weight.dtype), _native.stream(x.device))
    return s, y
