"""Sigmoid-gated product ``x * sigmoid(gate)`` on the HIP library.

Reference: qwen_triton/kernels/sigmoid_mul.py:35-195 (torch fallback :35-50,
kernels :66-120, autograd :140-177, public op :180-195).
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, needs_grad, Unsupported

_GUARD = OpGuard("Sigmoid-mul")


def _torch_sigmoid_mul(x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    return x * torch.sigmoid(gate)


def _torch_sigmoid_mul_backward(x: torch.Tensor, gate: torch.Tensor, grad_output: torch.Tensor):
    xf = x.to(torch.float32)
    gf = gate.to(torch.float32)
    go = grad_output.to(torch.float32)
    sig = torch.sigmoid(gf)
    return (go * sig).to(x.dtype), (go * xf * sig * (1.0 - sig)).to(gate.dtype)


def _native_sigmoid_mul(x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    _native.require_device(x, gate)
    if x.shape != gate.shape or x.dtype != gate.dtype:
        raise Unsupported("sigmoid_mul kernel needs equal shapes and dtypes")
    xc, gc = x.contiguous(), gate.contiguous()
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _native.call("qh_sigmoid_mul_fwd", xc.data_ptr(), gc.data_ptr(), out.data_ptr(), out.numel(),
                 _native.dtype_code(x.dtype), _native.stream(x.device))
    return out


def _native_sigmoid_mul_backward(x: torch.Tensor, gate: torch.Tensor, grad_output: torch.Tensor):
    xc, gc, go = x.contiguous(), gate.contiguous(), grad_output.contiguous().to(x.dtype)
    dx = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    dg = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    _native.call("qh_sigmoid_mul_bwd", xc.data_ptr(), gc.data_ptr(), go.data_ptr(), dx.data_ptr(), dg.data_ptr(),
                 xc.numel(), _native.dtype_code(x.dtype), _native.stream(x.device))
    return dx, dg


class _SigmoidMulFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        ctx.save_for_backward(x, gate)
        return _native_sigmoid_mul(x, gate)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        x, gate = ctx.saved_tensors
        try:
            return _native_sigmoid_mul_backward(x, gate, grad_output)
        except Exception as exc:
            _GUARD.failed(exc, "backward kernel")
            return _torch_sigmoid_mul_backward(x, gate, grad_output)


def sigmoid_mul(x: torch.Tensor, gate: torch.Tensor, use_triton: bool | None = None) -> torch.Tensor:
    if not _GUARD.use_native(use_triton, x, gate):
        return _torch_sigmoid_mul(x, gate)
    if x.shape != gate.shape:
        gate = gate.expand_as(x)
    try:
        if needs_grad(x, gate):
            return _SigmoidMulFunction.apply(x, gate)
        return _native_sigmoid_mul(x, gate)
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_sigmoid_mul(x, gate)
