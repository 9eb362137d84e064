"""Row softmax over the last dimension (MoE router) on the HIP library.

Reference: qwen_triton/kernels/softmax.py:35-184 (torch fallbacks :35-41,
kernels :56-127, autograd :138-166, public op :169-184).
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, needs_grad

_GUARD = OpGuard("Softmax")


def _torch_softmax(x: torch.Tensor) -> torch.Tensor:
    return torch.softmax(x, dim=-1)


def _torch_softmax_backward(output: torch.Tensor, grad_output: torch.Tensor) -> torch.Tensor:
    s = (grad_output * output).sum(dim=-1, keepdim=True)
    return output * (grad_output - s)


def _native_softmax(x: torch.Tensor) -> torch.Tensor:
    _native.require_device(x)
    xc = x.contiguous()
    cols = x.shape[-1] if x.dim() else 1
    rows = xc.numel() // cols if cols else 0
    out = torch.empty(xc.shape, dtype=x.dtype, device=x.device)
    _native.call("qh_softmax_fwd", xc.data_ptr(), out.data_ptr(), rows, cols, _native.dtype_code(x.dtype),
                 _native.stream(x.device))
    return out


def _native_softmax_backward(out: torch.Tensor, grad_output: torch.Tensor) -> torch.Tensor:
    y = out.contiguous()
    g = grad_output.contiguous().to(y.dtype)
    cols = y.shape[-1]
    rows = y.numel() // cols if cols else 0
    gx = torch.empty(y.shape, dtype=y.dtype, device=y.device)
    _native.call("qh_softmax_bwd", y.data_ptr(), g.data_ptr(), gx.data_ptr(), rows, cols,
                 _native.dtype_code(y.dtype), _native.stream(y.device))
    return gx


class _SoftmaxFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor) -> torch.Tensor:
        out = _native_softmax(x)
        ctx.save_for_backward(out)
        return out

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        (out,) = ctx.saved_tensors
        try:
            return (_native_softmax_backward(out, grad_output),)
        except Exception as exc:
            _GUARD.failed(exc, "backward kernel")
            return (_torch_softmax_backward(out, grad_output),)


def triton_softmax(x: torch.Tensor, use_triton: bool | None = None) -> torch.Tensor:
    if not _GUARD.use_native(use_triton, x):
        return _torch_softmax(x)
    try:
        if needs_grad(x):
            return _SoftmaxFunction.apply(x)
        return _native_softmax(x)
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_softmax(x)
