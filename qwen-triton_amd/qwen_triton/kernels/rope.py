"""Rotate-half rotary position embedding on the HIP library.

Reference: qwen_triton/kernels/rope.py:59-300 (torch fallback :59-73, kernel
:78-120, backend resolution :123-128, launcher :131-162, backward :165-203,
backend pair dispatch :206-250, autograd :253-283, public op :286-300).

Backends keep the reference's names: ``triton`` (this library's kernel called
directly), ``cuda_op`` (the same kernel behind the registered
``torch.ops.qwen_triton.rope_tensor_forward`` custom op), ``auto`` (custom op,
then direct) and ``torch``. Unlike the reference kernel (rope.py:102-114), a
cos/sin batch of 1 broadcasts over the input batch.
"""
from __future__ import annotations

import os
import warnings

import torch

from .. import _native
from ..ops import apply_rope_cuda_op, get_rope_cuda_op_error, load_rope_cuda_op
from ._common import OpGuard

_GUARD = OpGuard("RoPE")
_CUDA_OP_FALLBACK_WARNED = False
_TORCH_FALLBACK_WARNED = False


def _warn_cuda_op_fallback_once(exc: BaseException) -> None:
    global _CUDA_OP_FALLBACK_WARNED
    if _CUDA_OP_FALLBACK_WARNED:
        return
    _CUDA_OP_FALLBACK_WARNED = True
    warnings.warn(
        f"[Qwen-Triton fallback] RoPE custom op unavailable ({exc.__class__.__name__}: {exc}). "
        "Using the direct HIP kernel.",
        RuntimeWarning,
        stacklevel=3,
    )


def _warn_torch_fallback_once(reason: str) -> None:
    global _TORCH_FALLBACK_WARNED
    if _TORCH_FALLBACK_WARNED:
        return
    _TORCH_FALLBACK_WARNED = True
    warnings.warn(f"[Qwen-Triton fallback] {reason}. Using torch fallback.", RuntimeWarning, stacklevel=3)


def _torch_apply_rope_tensor(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    rotary_dim = cos.shape[-1]
    half = rotary_dim // 2
    x_rot, x_pass = x[..., :rotary_dim], x[..., rotary_dim:]
    c = cos.unsqueeze(1)[..., :half]
    s = sin.unsqueeze(1)[..., :half]
    x1, x2 = x_rot[..., :half], x_rot[..., half:rotary_dim]
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s, x_pass), dim=-1)


def _torch_apply_rope(q, k, cos, sin):
    return _torch_apply_rope_tensor(q, cos, sin), _torch_apply_rope_tensor(k, cos, sin)


def rope_tensor(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, neg_sin: bool = False) -> torch.Tensor:
    """One HIP launch of rotate-half RoPE; returns a contiguous [B, H, S, D] tensor."""
    _native.require_device(x, cos, sin)
    if x.dim() != 4 or cos.dim() != 3 or sin.shape != cos.shape:
        raise ValueError("rope expects x [B,H,S,D] and cos/sin [B or 1, S, rotary_dim]")
    B, H, S, D = x.shape
    rot = cos.shape[-1]
    if cos.shape[1] != S or rot > D or rot % 2:
        raise ValueError(f"rope shape mismatch: x {tuple(x.shape)} cos {tuple(cos.shape)}")
    if cos.shape[0] not in (1, B):
        raise ValueError(f"rope cos/sin batch {cos.shape[0]} must be 1 or {B}")
    if sin.stride() != cos.stride():
        sin = sin.contiguous()
        cos = cos.contiguous()
    out = torch.empty((B, H, S, D), dtype=x.dtype, device=x.device)
    _native.call("qh_rope", x.data_ptr(), *x.stride(), cos.data_ptr(), sin.data_ptr(), *cos.stride(),
                 cos.shape[0], out.data_ptr(), B, H, S, D, rot, int(neg_sin), _native.dtype_code(x.dtype),
                 _native.dtype_code(cos.dtype), _native.stream(x.device))
    return out


def _resolve_backend(use_triton: bool | None, backend: str | None) -> str:
    if backend is None:
        if use_triton is False:
            return "torch"
        return os.environ.get("QWEN_TRITON_ROPE_BACKEND", "triton").lower()
    return backend.lower()


def _apply_rope_grad_tensor(grad, cos, sin, backend: str, strict: bool) -> torch.Tensor:
    if backend == "cuda_op" and grad.is_cuda:
        if load_rope_cuda_op(verbose=os.environ.get("QWEN_TRITON_BUILD_VERBOSE") == "1"):
            try:
                return torch.ops.qwen_triton.rope_tensor_forward(grad.contiguous(), cos, torch.neg(sin))
            except Exception as exc:
                if strict:
                    raise RuntimeError("RoPE custom op backward failed and strict mode is enabled.") from exc
                _warn_cuda_op_fallback_once(exc)
        elif strict:
            raise RuntimeError("RoPE custom op failed to load and strict mode is enabled.") from get_rope_cuda_op_error()

    if backend in {"triton", "cuda_op"} and grad.is_cuda and _GUARD.runtime_ok and _native.available():
        try:
            return rope_tensor(grad, cos, sin, neg_sin=True)
        except Exception as exc:
            _GUARD.runtime_ok = False
            if strict:
                raise RuntimeError("RoPE HIP backward failed and strict mode is enabled.") from exc
            _GUARD.failed(exc, "backward kernel")

    if strict and backend in {"triton", "cuda_op"} and grad.is_cuda:
        raise RuntimeError("RoPE backward fast path is unavailable and strict mode is enabled.")
    if grad.is_cuda and backend != "torch":
        _warn_torch_fallback_once("RoPE backward fast path is unavailable")
    return _torch_apply_rope_tensor(grad, cos, torch.neg(sin))


def _apply_rope_backend_pair(q, k, cos, sin, resolved_backend: str, strict: bool):
    if resolved_backend == "torch":
        return _torch_apply_rope(q, k, cos, sin), "torch"
    if resolved_backend not in {"auto", "cuda_op", "triton"}:
        raise ValueError(f"Unsupported RoPE backend: {resolved_backend}")

    if resolved_backend in {"auto", "cuda_op"} and q.is_cuda and k.is_cuda:
        if load_rope_cuda_op(verbose=os.environ.get("QWEN_TRITON_BUILD_VERBOSE") == "1"):
            try:
                return apply_rope_cuda_op(q, k, cos, sin), "cuda_op"
            except Exception as exc:
                if strict and resolved_backend == "cuda_op":
                    raise RuntimeError("RoPE custom op failed and strict mode is enabled.") from exc
                _warn_cuda_op_fallback_once(exc)
        elif resolved_backend == "cuda_op":
            error = get_rope_cuda_op_error()
            if strict:
                raise RuntimeError("RoPE custom op failed to load and strict mode is enabled.") from error
            _warn_cuda_op_fallback_once(error or RuntimeError("unknown custom op load failure"))

    on_gpu = q.is_cuda and k.is_cuda
    if on_gpu and _GUARD.runtime_ok and not _native.available():
        raise RuntimeError(f"RoPE: the HIP operator library could not be loaded: {_native.load_error()!r}")
    if not (on_gpu and _GUARD.runtime_ok):
        if strict and resolved_backend in {"triton", "auto", "cuda_op"}:
            raise RuntimeError("RoPE HIP kernel is unavailable and strict mode is enabled.")
        if on_gpu:
            _warn_torch_fallback_once("RoPE HIP kernel is unavailable")
        return _torch_apply_rope(q, k, cos, sin), "torch"

    try:
        return (rope_tensor(q, cos, sin), rope_tensor(k, cos, sin)), "triton"
    except Exception as exc:
        _GUARD.runtime_ok = False
        if strict:
            raise RuntimeError("RoPE HIP kernel failed and strict mode is enabled.") from exc
        _GUARD.failed(exc)
        return _torch_apply_rope(q, k, cos, sin), "torch"


class _RoPEPairFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, cos, sin, resolved_backend: str, strict: bool):
        ctx.save_for_backward(cos, sin)
        outputs, actual_backend = _apply_rope_backend_pair(q, k, cos, sin, resolved_backend, strict)
        ctx.actual_backend = actual_backend
        ctx.strict = strict
        return outputs

    @staticmethod
    def backward(ctx, grad_q, grad_k):
        cos, sin = ctx.saved_tensors
        gq = _apply_rope_grad_tensor(grad_q, cos, sin, ctx.actual_backend, ctx.strict) if ctx.needs_input_grad[0] else None
        gk = _apply_rope_grad_tensor(grad_k, cos, sin, ctx.actual_backend, ctx.strict) if ctx.needs_input_grad[1] else None
        return gq, gk, None, None, None, None


def apply_rope(q, k, cos, sin, use_triton: bool | None = None, backend: str | None = None):
    resolved_backend = _resolve_backend(use_triton, backend)
    strict = os.environ.get("QWEN_TRITON_STRICT") == "1"
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad):
        return _RoPEPairFunction.apply(q, k, cos, sin, resolved_backend, strict)
    outputs, _ = _apply_rope_backend_pair(q, k, cos, sin, resolved_backend, strict)
    return outputs
