"""RoPE custom op ``torch.ops.qwen_triton.rope_tensor_forward`` backed by HIP.

Reference: qwen_triton/ops/rope_cuda.py:1-89 (JIT build + load :32-58, autograd
wrapper :61-80, pair API :83-89) and the op schema of
qwen_triton/csrc/rope_op.cpp:17-23. Here "loading" the op means loading
libqwen_hip.so and registering the schema with a CUDA-key implementation that
calls the library's ``qh_rope``; nothing is compiled at run time.
"""
from __future__ import annotations

import torch

from .. import _native

_LOAD_ATTEMPTED = False
_LOAD_ERROR: Exception | None = None
_LOADED = False
_TORCH_LIB = None


def _rope_tensor_forward_impl(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    from ..kernels.rope import rope_tensor

    return rope_tensor(x, cos, sin)


def get_rope_cuda_op_error() -> Exception | None:
    return _LOAD_ERROR


def load_rope_cuda_op(verbose: bool = False) -> bool:
    global _LOAD_ATTEMPTED, _LOAD_ERROR, _LOADED, _TORCH_LIB
    if _LOADED:
        return True
    if _LOAD_ATTEMPTED and _LOAD_ERROR is not None:
        return False
    _LOAD_ATTEMPTED = True
    try:
        _native.lib()
        lib = torch.library.Library("qwen_triton", "DEF")
        lib.define("rope_tensor_forward(Tensor x, Tensor cos, Tensor sin) -> Tensor")
        lib.impl("rope_tensor_forward", _rope_tensor_forward_impl, "CUDA")
        _TORCH_LIB = lib
    except Exception as exc:
        _LOAD_ERROR = exc
        if verbose:
            print(f"[qwen_triton] RoPE custom op registration failed: {exc!r}")
        return False
    _LOAD_ERROR = None
    _LOADED = True
    return True


class _RopeTensorCudaFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        if not load_rope_cuda_op():
            raise RuntimeError("Qwen RoPE custom op is unavailable.") from get_rope_cuda_op_error()
        ctx.save_for_backward(cos, sin)
        return torch.ops.qwen_triton.rope_tensor_forward(x, cos, sin)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        if grad_output is None:
            return None, None, None
        from ..kernels.rope import rope_tensor

        cos, sin = ctx.saved_tensors
        return rope_tensor(grad_output, cos, sin, neg_sin=True), None, None


def apply_rope_cuda_op(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    return _RopeTensorCudaFunction.apply(q, cos, sin), _RopeTensorCudaFunction.apply(k, cos, sin)
