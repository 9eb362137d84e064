"""Residual add ``x + residual`` on the HIP library.

Reference: qwen_triton/kernels/residual_add.py:35-101 (torch fallback :35-36,
kernel :50-60, autograd :76-83, public op :86-101).
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, needs_grad, Unsupported

_GUARD = OpGuard("ResidualAdd")


def _torch_residual_add(x: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    return x + residual


def _native_residual_add(x: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    _native.require_device(x, residual)
    if x.shape != residual.shape or x.dtype != residual.dtype:
        raise Unsupported("residual_add kernel needs equal shapes and dtypes")
    xc, rc = x.contiguous(), residual.contiguous()
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _native.call("qh_add", xc.data_ptr(), rc.data_ptr(), out.data_ptr(), out.numel(),
                 _native.dtype_code(x.dtype), _native.stream(x.device))
    return out


class _ResidualAddFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        return _native_residual_add(x, residual)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        return grad_output, grad_output


def residual_add(x: torch.Tensor, residual: torch.Tensor, use_triton: bool | None = None) -> torch.Tensor:
    if not _GUARD.use_native(use_triton, x, residual):
        return _torch_residual_add(x, residual)
    if x.shape != residual.shape or x.dtype != residual.dtype:
        return _torch_residual_add(x, residual)  # broadcasting / promotion: plain torch semantics
    try:
        if needs_grad(x, residual):
            return _ResidualAddFunction.apply(x, residual)
        return _native_residual_add(x, residual)
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_residual_add(x, residual)
