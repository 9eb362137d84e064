"""KV-cache write-by-position and append on the HIP library.

Reference: qwen_triton/kernels/cache.py:37-181 (append kernel :37-69, write
kernel :72-98, ``append_attention_kv`` :101-139, ``write_attention_kv``
:142-181).
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, Unsupported

_GUARD = OpGuard("KV cache")


def append_attention_kv(prefix: torch.Tensor | None, suffix: torch.Tensor) -> torch.Tensor:
    if prefix is None:
        return suffix
    if not (prefix.is_cuda and suffix.is_cuda) or prefix.dim() != 4 or suffix.dim() != 4:
        return torch.cat((prefix, suffix), dim=-2)
    if not _GUARD.use_native(None, prefix, suffix):
        return torch.cat((prefix, suffix), dim=-2)
    try:
        B, H, so, D = prefix.shape
        sn = suffix.shape[-2]
        if suffix.shape[:2] != prefix.shape[:2] or suffix.shape[-1] != D or suffix.dtype != prefix.dtype:
            raise Unsupported("append_attention_kv shape/dtype mismatch")
        pre, suf = prefix.contiguous(), suffix.contiguous()
        out = torch.empty((B, H, so + sn, D), dtype=prefix.dtype, device=prefix.device)
        _native.call("qh_kv_append", pre.data_ptr(), suf.data_ptr(), out.data_ptr(), B, H, so, sn, D,
                     _native.dtype_code(prefix.dtype), _native.stream(prefix.device))
        return out
    except Exception as exc:
        _GUARD.failed(exc)
        return torch.cat((prefix, suffix), dim=-2)


def write_attention_kv(cache: torch.Tensor, values: torch.Tensor, positions: torch.LongTensor) -> torch.Tensor:
    """``cache[:, :, positions, :] = values`` in place; returns ``cache``."""
    if values.numel() == 0:
        return cache
    positions = positions.to(device=cache.device, dtype=torch.long).contiguous()
    if not (cache.is_cuda and values.is_cuda and positions.is_cuda) or cache.dim() != 4 or values.dim() != 4:
        cache[:, :, positions, :] = values
        return cache
    if not _GUARD.use_native(None, cache, values):
        cache[:, :, positions, :] = values
        return cache
    try:
        B, H, S, D = values.shape
        if cache.shape[0] != B or cache.shape[1] != H or cache.shape[3] != D or positions.numel() != S:
            raise Unsupported(f"write_attention_kv shape mismatch: cache {tuple(cache.shape)} values {tuple(values.shape)}")
        if values.dtype != cache.dtype:
            values = values.to(cache.dtype)
        _native.call("qh_kv_write", cache.data_ptr(), *cache.stride(), values.data_ptr(), *values.stride(),
                     positions.data_ptr(), B, H, S, D, cache.shape[2], _native.dtype_code(cache.dtype),
                     _native.stream(cache.device))
    except Exception as exc:
        _GUARD.failed(exc)
        cache[:, :, positions, :] = values
    return cache
