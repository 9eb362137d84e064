"""Mean cross-entropy over 2-D logits with ``ignore_index`` on the HIP library.

Reference: qwen_triton/kernels/cross_entropy.py:35-226 (torch fallback :35-40,
forward kernel :55-95, backward kernel :108-139, forward launcher :142-161,
autograd :164-202, public op :205-226). The loss is
``sum(lse - logit[target]) / max(1, n_valid)`` in fp32 like the reference's
kernel path; unlike it, neither direction synchronises with the host: the valid
count and the upstream gradient stay on the device.
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, Unsupported

_GUARD = OpGuard("CrossEntropy")


def _torch_cross_entropy(logits: torch.Tensor, targets: torch.Tensor, ignore_index: int = -100) -> torch.Tensor:
    return torch.nn.functional.cross_entropy(logits, targets, ignore_index=ignore_index)


def _native_ce_forward(logits: torch.Tensor, targets: torch.Tensor, ignore_index: int):
    _native.require_device(logits, targets)
    if logits.dim() != 2:
        raise Unsupported("cross-entropy kernel expects 2-D logits [N, V]")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    tg = targets.contiguous().view(-1)
    if tg.dtype != torch.long:
        tg = tg.long()
    N, V = logits.shape
    if tg.numel() != N:
        raise Unsupported("targets must have one entry per logits row")
    dev = logits.device
    lse = torch.empty(N, dtype=torch.float32, device=dev)
    rows = torch.empty(N, dtype=torch.float32, device=dev)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    n_valid = torch.empty(1, dtype=torch.float32, device=dev)
    _native.call("qh_ce_fwd", logits.data_ptr(), logits.stride(0), tg.data_ptr(), lse.data_ptr(), rows.data_ptr(),
                 loss.data_ptr(), n_valid.data_ptr(), N, V, int(ignore_index), _native.dtype_code(logits.dtype),
                 _native.stream(dev))
    return loss, lse, n_valid, logits, tg


class _CrossEntropyFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits: torch.Tensor, targets: torch.Tensor, ignore_index: int) -> torch.Tensor:
        loss, lse, n_valid, lg, tg = _native_ce_forward(logits, targets, ignore_index)
        ctx.save_for_backward(lg, tg, lse, n_valid)
        ctx.ignore_index = ignore_index
        return loss

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        logits, targets, lse, n_valid = ctx.saved_tensors
        try:
            N, V = logits.shape
            gl = grad_output.detach().to(torch.float32).reshape(1).contiguous()
            grad_logits = torch.empty((N, V), dtype=logits.dtype, device=logits.device)
            _native.call("qh_ce_bwd", logits.data_ptr(), logits.stride(0), targets.data_ptr(), lse.data_ptr(),
                         gl.data_ptr(), n_valid.data_ptr(), grad_logits.data_ptr(), grad_logits.stride(0), N, V,
                         int(ctx.ignore_index), _native.dtype_code(logits.dtype), _native.stream(logits.device))
            return grad_logits, None, None
        except Exception as exc:
            _GUARD.failed(exc, "backward kernel")
            with torch.enable_grad():
                x = logits.detach().requires_grad_(True)
                loss = _torch_cross_entropy(x, targets, ctx.ignore_index)
                (g,) = torch.autograd.grad(loss, x, grad_output)
            return g, None, None


def triton_cross_entropy(
    logits: torch.Tensor,
    targets: torch.Tensor,
    ignore_index: int = -100,
    use_triton: bool | None = None,
) -> torch.Tensor:
    if not _GUARD.use_native(use_triton, logits, targets):
        return _torch_cross_entropy(logits, targets, ignore_index)
    try:
        if torch.is_grad_enabled() and logits.requires_grad:
            return _CrossEntropyFunction.apply(logits, targets, ignore_index)
        return _native_ce_forward(logits, targets, ignore_index)[0]
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_cross_entropy(logits, targets, ignore_index)
