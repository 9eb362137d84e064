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
from typing import Callable

import torch

from .. import _native
from ..ops import apply_rope_cuda_op, get_rope_cuda_op_error, load_rope_cuda_op
from ._common import OpGuard, Unsupported

_GUARD = OpGuard("RoPE")


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
        raise Unsupported("rope expects x [B,H,S,D] and cos/sin [B or 1, S, rotary_dim]")
    B, H, S, D = x.shape
    rot = cos.shape[-1]
    if cos.shape[1] != S or rot > D or rot % 2:
        raise Unsupported(f"rope shape mismatch: x {tuple(x.shape)} cos {tuple(cos.shape)}")
    if cos.shape[0] not in (1, B):
        raise Unsupported(f"rope cos/sin batch {cos.shape[0]} must be 1 or {B}")
    if sin.stride() != cos.stride():
        sin = sin.contiguous()
        cos = cos.contiguous()
    out = torch.empty((B, H, S, D), dtype=x.dtype, device=x.device)
    _native.call("qh_rope", x.data_ptr(), *x.stride(), cos.data_ptr(), sin.data_ptr(), *cos.stride(),
                 cos.shape[0], out.data_ptr(), B, H, S, D, rot, int(neg_sin), _native.dtype_code(x.dtype),
                 _native.dtype_code(cos.dtype), _native.stream(x.device))
    return out


# ---------------------------------------------------------------------------
# Backend routing.
#
# A requested backend names the accelerated routes to try, in order; torch
# always ends the list. Routes:
#   "custom_op"  torch.ops.qwen_triton.rope_tensor_forward, registered by
#                qwen_triton.ops (it calls the same HIP kernel);
#   "hip"        rope_tensor, the library kernel called directly.
# A route flagged `required` may not be skipped under QWEN_TRITON_STRICT=1: if
# it cannot run, or fails, the call raises RuntimeError. Otherwise the call
# moves on to the next route, with at most one RuntimeWarning per kind of
# hand-over in the process. The backward retraces the route the forward took.
# ---------------------------------------------------------------------------
_FORWARD_ROUTES: dict[str, tuple[tuple[str, bool], ...]] = {
    "torch": (),
    "triton": (("hip", True),),
    "cuda_op": (("custom_op", True), ("hip", True)),
    "auto": (("custom_op", False), ("hip", True)),
}
# what each route reports as the backend it ran (the reference's names)
_BACKEND_OF = {"custom_op": "cuda_op", "hip": "triton", "torch": "torch"}
_BACKWARD_ROUTES = {"cuda_op": _FORWARD_ROUTES["cuda_op"], "triton": _FORWARD_ROUTES["triton"], "torch": ()}

_HANDOVER_WARNED: set[str] = set()


def _warn_handover(kind: str, detail: str) -> None:
    if kind in _HANDOVER_WARNED:
        return
    _HANDOVER_WARNED.add(kind)
    nxt = "the direct HIP kernel" if kind == "custom_op" else "torch"
    warnings.warn(f"[Qwen-Triton fallback] RoPE {detail}. Using {nxt}.", RuntimeWarning, stacklevel=4)


def _resolve_backend(use_triton: bool | None, backend: str | None) -> str:
    """Requested backend: the explicit argument, else torch for use_triton=False, else
    QWEN_TRITON_ROPE_BACKEND (default "triton")."""
    if backend is not None:
        return backend.lower()
    if use_triton is False:
        return "torch"
    return os.environ.get("QWEN_TRITON_ROPE_BACKEND", "triton").lower()


def _on_gpu(*tensors: torch.Tensor) -> bool:
    return all(t.is_cuda for t in tensors)


def _custom_op_single(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    return torch.ops.qwen_triton.rope_tensor_forward(x, cos, sin)


def _route_unready(route: str, on_gpu: bool) -> str | None:
    """Why `route` cannot run now (None when it can)."""
    if not on_gpu:
        return "inputs are not on the GPU"
    if route == "custom_op":
        if load_rope_cuda_op(verbose=os.environ.get("QWEN_TRITON_BUILD_VERBOSE") == "1"):
            return None
        return f"custom op unavailable ({get_rope_cuda_op_error()!r})"
    if not _GUARD.runtime_ok:
        return "HIP kernel disabled after an earlier failure"
    if not _native.available():  # GPU inputs never fall back silently for a missing library
        raise RuntimeError(f"RoPE: the HIP operator library could not be loaded: {_native.load_error()!r}")
    return None


def _run_routes(routes, on_gpu: bool, strict: bool, attempt: Callable[[str], object], what: str):
    """Try `routes` in order; returns (result, route), or (None, "torch") when torch must compute it."""
    for route, required in routes:
        why = _route_unready(route, on_gpu)
        if why is not None:
            if strict and required:
                raise RuntimeError(f"RoPE {what}: {route} route unavailable ({why}) and strict mode is enabled.")
            if on_gpu and required and route == "custom_op":
                _warn_handover("custom_op", why)
            continue
        try:
            return attempt(route), route
        except Exception as exc:
            if route == "hip":
                _GUARD.failed(exc, what)  # sticky unless Unsupported; raises in strict mode
            elif strict and required:
                raise RuntimeError(f"RoPE {what}: custom op failed and strict mode is enabled.") from exc
            else:
                _warn_handover("custom_op", f"custom op failed ({exc.__class__.__name__}: {exc})")
    if on_gpu and routes:
        _warn_handover("torch", f"{what}: no accelerated route ran")
    return None, "torch"


def _apply_rope_backend_pair(q, k, cos, sin, requested: str, strict: bool):
    """Forward over the requested backend's routes; returns ((q_out, k_out), backend that ran)."""
    routes = _FORWARD_ROUTES.get(requested)
    if routes is None:
        raise ValueError(f"Unsupported RoPE backend: {requested}")

    def attempt(route: str):
        if route == "custom_op":
            return apply_rope_cuda_op(q, k, cos, sin)
        return rope_tensor(q, cos, sin), rope_tensor(k, cos, sin)

    out, route = _run_routes(routes, _on_gpu(q, k), strict, attempt, "kernel")
    if out is None:
        out = _torch_apply_rope(q, k, cos, sin)
    return out, _BACKEND_OF[route]


def _apply_rope_grad_tensor(grad, cos, sin, backend: str, strict: bool) -> torch.Tensor:
    """Backward of one tensor (RoPE with -sin, its exact transpose) over the forward's routes."""

    def attempt(route: str):
        if route == "custom_op":
            return _custom_op_single(grad.contiguous(), cos, torch.neg(sin))
        return rope_tensor(grad, cos, sin, neg_sin=True)

    out, _ = _run_routes(_BACKWARD_ROUTES[backend], _on_gpu(grad), strict, attempt, "backward kernel")
    return out if out is not None else _torch_apply_rope_tensor(grad, cos, torch.neg(sin))


class _RoPEPairFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, cos, sin, resolved_backend: str, strict: bool):
        (qo, ko), ran = _apply_rope_backend_pair(q, k, cos, sin, resolved_backend, strict)
        ctx.save_for_backward(cos, sin)
        ctx.ran, ctx.strict = ran, strict
        return qo, ko

    @staticmethod
    def backward(ctx, grad_q, grad_k):
        cos, sin = ctx.saved_tensors
        need_q, need_k = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        gq = _apply_rope_grad_tensor(grad_q, cos, sin, ctx.ran, ctx.strict) if need_q else None
        gk = _apply_rope_grad_tensor(grad_k, cos, sin, ctx.ran, ctx.strict) if need_k else None
        return gq, gk, None, None, None, None


def apply_rope(q, k, cos, sin, use_triton: bool | None = None, backend: str | None = None):
    requested = _resolve_backend(use_triton, backend)
    strict = os.environ.get("QWEN_TRITON_STRICT") == "1"
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad):
        return _RoPEPairFunction.apply(q, k, cos, sin, requested, strict)
    return _apply_rope_backend_pair(q, k, cos, sin, requested, strict)[0]
