"""MoE routing primitives on the HIP library: top-k, one-hot, index_add.

Reference: qwen_triton/kernels/moe_routing.py:1-343 (top-k kernels :45-116,
launcher :119-144, top-k autograd :147-162, one-hot :171-200, index_add
:207-255, public ops :258-343).

* ``triton_topk`` sorts each row's k largest values descending with ties broken
  towards the lower index (the rule of moe_routing.py:96-116), without cloning
  or mutating the input.
* ``triton_index_add`` is deterministic: sources are grouped per destination
  row by a stable sort and summed in source order in fp32 (one rounding per
  row) instead of racing atomics.
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, needs_grad, Unsupported

_GUARD = OpGuard("MoE routing")


def _torch_topk(x: torch.Tensor, k: int):
    return torch.topk(x, k, dim=-1)


def _torch_one_hot(indices: torch.Tensor, num_classes: int) -> torch.Tensor:
    return torch.nn.functional.one_hot(indices, num_classes)


def _torch_index_add(target: torch.Tensor, source: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    target.index_add_(0, index, source)
    return target


def _native_topk(x: torch.Tensor, k: int):
    _native.require_device(x)
    if x.dim() != 2:
        raise Unsupported("top-k kernel expects a 2-D [N, C] input")
    xc = x.contiguous()
    N, C = xc.shape
    vals = torch.empty((N, k), dtype=x.dtype, device=x.device)
    idx = torch.empty((N, k), dtype=torch.int64, device=x.device)
    _native.call("qh_topk", xc.data_ptr(), vals.data_ptr(), idx.data_ptr(), N, C, int(k),
                 _native.dtype_code(x.dtype), _native.stream(x.device))
    return vals, idx


class _TopkFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, k: int):
        vals, idxs = _native_topk(x, k)
        ctx.save_for_backward(idxs)
        ctx.input_shape = x.shape
        ctx.mark_non_differentiable(idxs)
        return vals, idxs

    @staticmethod
    def backward(ctx, grad_vals: torch.Tensor, grad_idxs: torch.Tensor | None):
        (idxs,) = ctx.saved_tensors
        grad_x = torch.zeros(ctx.input_shape, device=grad_vals.device, dtype=grad_vals.dtype)
        grad_x.scatter_add_(1, idxs, grad_vals)
        return grad_x, None


def triton_topk(x: torch.Tensor, k: int, use_triton: bool | None = None):
    if not _GUARD.use_native(use_triton, x):
        return _torch_topk(x, k)
    try:
        if needs_grad(x):
            return _TopkFunction.apply(x, k)
        return _native_topk(x, k)
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_topk(x, k)


def _native_one_hot(indices: torch.Tensor, num_classes: int) -> torch.Tensor:
    _native.require_device(indices)
    flat = indices.contiguous().view(-1)
    if flat.dtype != torch.long:
        flat = flat.long()
    N = flat.numel()
    out = torch.empty((N, num_classes), dtype=torch.int64, device=indices.device)
    _native.call("qh_one_hot", flat.data_ptr(), out.data_ptr(), N, int(num_classes), _native.stream(indices.device))
    return out.view(*indices.shape, num_classes)


def triton_one_hot(indices: torch.Tensor, num_classes: int, use_triton: bool | None = None) -> torch.Tensor:
    if not _GUARD.use_native(use_triton, indices):
        return _torch_one_hot(indices, num_classes)
    try:
        return _native_one_hot(indices, num_classes)
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_one_hot(indices, num_classes)


def _native_index_add(target: torch.Tensor, source: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """In place on ``target``; rows of ``index`` outside [0, len(target)) are skipped."""
    _native.require_device(target, source, index)
    if target.dim() != 2 or source.dim() != 2 or target.shape[1] != source.shape[1]:
        raise Unsupported("index_add kernel expects 2-D target/source with equal row width")
    if target.stride(1) != 1:
        raise Unsupported("index_add kernel needs a row-major target")
    src = source if source.stride(1) == 1 else source.contiguous()
    if src.dtype != target.dtype:
        src = src.to(target.dtype)
    idx = index.contiguous().view(-1)
    if idx.dtype != torch.long:
        idx = idx.long()
    n_src = src.shape[0]
    if idx.numel() != n_src:
        raise Unsupported("index must have one entry per source row")
    ws = _native.workspace(_native.call("qh_index_add_workspace", n_src), target.device)
    _native.call("qh_index_add", target.data_ptr(), target.stride(0), src.data_ptr(), src.stride(0), idx.data_ptr(),
                 n_src, target.shape[0], target.shape[1], ws.data_ptr(), ws.numel(),
                 _native.dtype_code(target.dtype), _native.stream(target.device))
    return target


class _IndexAddFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, target: torch.Tensor, source: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
        ctx.save_for_backward(index)
        out = target.clone()
        _native_index_add(out, source, index)
        return out

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        (index,) = ctx.saved_tensors
        return grad_output, grad_output[index], None


def triton_index_add(target: torch.Tensor, source: torch.Tensor, index: torch.Tensor, use_triton: bool | None = None):
    if not _GUARD.use_native(use_triton, target):
        return _torch_index_add(target, source, index)
    try:
        if needs_grad(target, source):
            return _IndexAddFunction.apply(target, source, index)
        return _native_index_add(target, source, index)
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_index_add(target, source, index)
