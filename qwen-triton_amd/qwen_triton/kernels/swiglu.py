"""SiLU-gated product ``silu(gate) * up`` (SwiGLU) on the HIP library.

Reference: qwen_triton/kernels/swiglu.py:35-190 (torch fallback :35-51,
kernels :84-132, autograd :135-172, public op :175-190).
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, needs_grad, Unsupported

_GUARD = OpGuard("SiLU-mul")


def _torch_silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    return torch.nn.functional.silu(gate) * up


def _torch_silu_mul_backward(gate: torch.Tensor, up: torch.Tensor, grad_output: torch.Tensor):
    g = gate.to(torch.float32)
    u = up.to(torch.float32)
    go = grad_output.to(torch.float32)
    sig = torch.sigmoid(g)
    grad_gate = go * u * sig * (1.0 + g * (1.0 - sig))
    grad_up = go * g * sig
    return grad_gate.to(gate.dtype), grad_up.to(up.dtype)


def _check(gate: torch.Tensor, up: torch.Tensor) -> None:
    _native.require_device(gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise Unsupported("silu_mul kernel needs equal shapes and dtypes")


def _native_silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    _check(gate, up)
    g, u = gate.contiguous(), up.contiguous()
    out = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    _native.call("qh_silu_mul_fwd", g.data_ptr(), u.data_ptr(), out.data_ptr(), out.numel(),
                 _native.dtype_code(gate.dtype), _native.stream(gate.device))
    return out


def _native_silu_mul_backward(gate: torch.Tensor, up: torch.Tensor, grad_output: torch.Tensor):
    g, u, go = gate.contiguous(), up.contiguous(), grad_output.contiguous().to(gate.dtype)
    dg = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    du = torch.empty(up.shape, dtype=up.dtype, device=up.device)
    _native.call("qh_silu_mul_bwd", g.data_ptr(), u.data_ptr(), go.data_ptr(), dg.data_ptr(), du.data_ptr(),
                 g.numel(), _native.dtype_code(gate.dtype), _native.stream(gate.device))
    return dg, du


class _SiLUMulFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
        ctx.save_for_backward(gate, up)
        return _native_silu_mul(gate, up)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        gate, up = ctx.saved_tensors
        try:
            return _native_silu_mul_backward(gate, up, grad_output)
        except Exception as exc:
            _GUARD.failed(exc, "backward kernel")
            return _torch_silu_mul_backward(gate, up, grad_output)


def silu_mul(gate: torch.Tensor, up: torch.Tensor, use_triton: bool | None = None) -> torch.Tensor:
    if not _GUARD.use_native(use_triton, gate, up):
        return _torch_silu_mul(gate, up)
    try:
        if needs_grad(gate, up):
            return _SiLUMulFunction.apply(gate, up)
        return _native_silu_mul(gate, up)
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_silu_mul(gate, up)
