"""Embedding gather and its deterministic backward on the HIP library.

Reference: qwen_triton/kernels/embedding.py:35-186 (torch fallback :35-36,
kernels :50-94, forward launcher :97-112, autograd :115-163, public op
:166-186). The backward replaces fp32 atomics into a dense [V, H] buffer with a
stable radix sort of token ids, then writes every weight-gradient row once:
zeros, or the ordered fp32 sum of the rows of the tokens that hit it.
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, needs_grad, Unsupported

_GUARD = OpGuard("Embedding")


def _torch_embedding(input_ids: torch.Tensor, weight: torch.Tensor, padding_idx: int | None = None) -> torch.Tensor:
    return torch.nn.functional.embedding(input_ids, weight, padding_idx=padding_idx)


def _native_embedding(input_ids: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    _native.require_device(input_ids, weight)
    if weight.dim() != 2 or weight.stride(1) != 1:
        raise Unsupported("embedding weight must be a row-major [V, H] matrix")
    ids = input_ids.contiguous().view(-1)
    if ids.dtype != torch.long:
        ids = ids.long()
    n, (V, Hd) = ids.numel(), weight.shape
    out = torch.empty((n, Hd), dtype=weight.dtype, device=weight.device)
    _native.call("qh_embedding_fwd", ids.data_ptr(), weight.data_ptr(), weight.stride(0), out.data_ptr(), n, V, Hd,
                 _native.dtype_code(weight.dtype), _native.stream(weight.device))
    return out.view(*input_ids.shape, Hd)


def _native_embedding_backward(input_ids, grad_output, num_embeddings, embed_dim, padding_idx, weight_dtype, device):
    ids = input_ids.contiguous().view(-1)
    if ids.dtype != torch.long:
        ids = ids.long()
    g = grad_output.contiguous().view(-1, embed_dim)
    n = ids.numel()
    gw = torch.empty((num_embeddings, embed_dim), dtype=weight_dtype, device=device)
    ws = _native.workspace(_native.call("qh_embedding_bwd_workspace", n, num_embeddings), device)
    pad = -1 if padding_idx is None else int(padding_idx) % num_embeddings
    _native.call("qh_embedding_bwd", ids.data_ptr(), g.data_ptr(), gw.data_ptr(), ws.data_ptr(), ws.numel(), n,
                 num_embeddings, embed_dim, pad, _native.dtype_code(g.dtype), _native.dtype_code(weight_dtype),
                 _native.stream(device))
    return gw


class _EmbeddingFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, input_ids: torch.Tensor, weight: torch.Tensor, padding_idx: int | None) -> torch.Tensor:
        ctx.save_for_backward(input_ids)
        ctx.num_embeddings, ctx.embed_dim = weight.shape
        ctx.padding_idx = padding_idx
        ctx.weight_dtype = weight.dtype
        ctx.weight_device = weight.device
        return _native_embedding(input_ids, weight)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        (input_ids,) = ctx.saved_tensors
        try:
            gw = _native_embedding_backward(input_ids, grad_output, ctx.num_embeddings, ctx.embed_dim,
                                            ctx.padding_idx, ctx.weight_dtype, ctx.weight_device)
        except Exception as exc:
            _GUARD.failed(exc, "backward kernel")
            ids = input_ids.reshape(-1)
            g = grad_output.reshape(-1, ctx.embed_dim)
            gw = torch.zeros((ctx.num_embeddings, ctx.embed_dim), device=ctx.weight_device, dtype=torch.float32)
            gw.index_add_(0, ids, g.float())
            if ctx.padding_idx is not None:
                gw[ctx.padding_idx] = 0
            gw = gw.to(ctx.weight_dtype)
        return None, gw, None


def triton_embedding(
    input_ids: torch.Tensor,
    weight: torch.Tensor,
    padding_idx: int | None = None,
    use_triton: bool | None = None,
) -> torch.Tensor:
    if not _GUARD.use_native(use_triton, weight):
        return _torch_embedding(input_ids, weight, padding_idx)
    try:
        if needs_grad(weight):
            return _EmbeddingFunction.apply(input_ids, weight, padding_idx)
        return _native_embedding(input_ids, weight)
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_embedding(input_ids, weight, padding_idx)
