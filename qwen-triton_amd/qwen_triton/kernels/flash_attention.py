"""Flash attention (forward, backward, single-query decode) on the HIP library.

Reference: qwen_triton/kernels/flash_attention.py:35-433 (SDPA fallback :35-49,
forward kernel :54-152, backward kernels :155-277, launchers :280-367, autograd
:370-406, public op :409-433).

``triton_flash_attention`` keeps the reference contract: q [B,Hq,Sq,D], k/v
[B,Hkv,Sk,D], GQA through ``num_kv_groups``, causal masking aligned top-left
(key j visible to query i iff j <= i), LSE saved for the backward. Two
extensions are used by the model layer only: ``causal_offset`` (bottom-right
alignment for prefill on top of a cache) and the split-KV decode kernel for a
single query over a long cache.
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, Unsupported

_GUARD = OpGuard("FlashAttention")


def _torch_flash_attention(q, k, v, scale: float, is_causal: bool = True, num_kv_groups: int = 1) -> torch.Tensor:
    if num_kv_groups > 1:
        B, nkv, S, D = k.shape
        k = k[:, :, None].expand(B, nkv, num_kv_groups, S, D).reshape(B, nkv * num_kv_groups, S, D)
        v = v[:, :, None].expand(B, nkv, num_kv_groups, S, D).reshape(B, nkv * num_kv_groups, S, D)
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=None, dropout_p=0.0,
                                                            is_causal=is_causal, scale=scale)


def _torch_attention_offset(q, k, v, scale: float, causal: bool, num_kv_groups: int, causal_offset: int):
    """Torch attention with the kernels' mask rule: key j visible to query i iff j <= i + causal_offset
    (offset 0 is SDPA's top-left ``is_causal``)."""
    if not causal or causal_offset == 0:
        return _torch_flash_attention(q, k, v, scale, causal, num_kv_groups)
    if num_kv_groups > 1:
        k = k.repeat_interleave(num_kv_groups, dim=1)
        v = v.repeat_interleave(num_kv_groups, dim=1)
    sq, sk = q.shape[2], k.shape[2]
    keep = (torch.arange(sk, device=q.device)[None, :]
            <= torch.arange(sq, device=q.device)[:, None] + causal_offset)
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=keep, dropout_p=0.0, scale=scale)


def _unit_last(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def _check(q, k, v, num_kv_groups):
    _native.require_device(q, k, v)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise Unsupported("flash attention expects 4-D [B, H, S, D] tensors")
    if k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[3] != k.shape[3]:
        raise Unsupported(f"flash attention shape mismatch q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    if q.shape[1] != k.shape[1] * num_kv_groups:
        raise Unsupported(f"q heads {q.shape[1]} != kv heads {k.shape[1]} x groups {num_kv_groups}")
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise Unsupported("flash attention kernels need bf16, fp16 or fp32 q/k/v of one dtype")


def pack_key_bits(key_valid: torch.Tensor) -> torch.Tensor:
    """[B, Sk] 0/1 key validity -> int64 [B, ceil(Sk / 64)] words, bit j % 64 of word j // 64 set
    when key j may be attended (the layout ``qh_flash_fwd_masked`` reads)."""
    B, sk = key_valid.shape
    words = (sk + 63) // 64
    bits = torch.zeros((B, words * 64), dtype=torch.int64, device=key_valid.device)
    bits[:, :sk] = (key_valid != 0).to(torch.int64)
    shifts = torch.arange(64, dtype=torch.int64, device=key_valid.device)
    # distinct powers of two: the sum is the OR (bit 63 wraps to the sign bit, as intended)
    return (bits.view(B, words, 64) << shifts).sum(dim=-1)


def flash_forward(q, k, v, scale: float, causal: bool, num_kv_groups: int, causal_offset: int = 0,
                  need_lse: bool = True, seq_major: bool = False, key_bits: torch.Tensor | None = None,
                  window: int = 0):
    """Launch the forward kernel; returns (out [B,Hq,Sq,D], lse [B,Hq,Sq] fp32 or None). ``out`` is
    contiguous, or with ``seq_major`` the [B,Hq,Sq,D] view of a [B,Sq,Hq,D] buffer (the rows the
    output projection reads, written in place by the kernel). ``key_bits`` (from ``pack_key_bits``)
    and ``window`` (> 0: key j hidden from query i when j <= i + causal_offset - window) select the
    masked kernel, bf16/f16 only."""
    _check(q, k, v, num_kv_groups)
    masked = key_bits is not None or window > 0
    if masked and q.dtype == torch.float32:
        raise Unsupported("the masked flash kernel takes bf16/fp16 q/k/v")
    q, k, v = _unit_last(q), _unit_last(k), _unit_last(v)
    B, Hq, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    if seq_major:
        out = torch.empty((B, Sq, Hq, D), dtype=q.dtype, device=q.device).permute(0, 2, 1, 3)
    else:
        out = torch.empty((B, Hq, Sq, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, Hq, Sq), dtype=torch.float32, device=q.device) if need_lse else None
    args = (q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
            v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), out.data_ptr(), out.stride(0), out.stride(1),
            out.stride(2), None if lse is None else lse.data_ptr(), B, Hq, Hkv, Sq, Sk, D, float(scale),
            int(bool(causal)), int(causal_offset))
    if masked:
        if key_bits is not None:
            if (key_bits.dtype != torch.int64 or key_bits.dim() != 2 or key_bits.shape[0] != B
                    or key_bits.shape[1] < (Sk + 63) // 64 or key_bits.stride(1) != 1
                    or key_bits.device != q.device):
                raise Unsupported(f"key_bits must be int64 [B, >= ceil(Sk / 64)] on {q.device}")
        _native.call("qh_flash_fwd_masked", *args, None if key_bits is None else key_bits.data_ptr(),
                     0 if key_bits is None else key_bits.stride(0), int(window), _native.dtype_code(q.dtype),
                     _native.stream(q.device))
    else:
        _native.call("qh_flash_fwd", *args, _native.dtype_code(q.dtype), _native.stream(q.device))
    return out, lse


def attention_rows(q, k, v, scale: float, num_kv_groups: int, causal_offset: int = 0,
                   key_bits: torch.Tensor | None = None, window: int = 0) -> torch.Tensor | None:
    """Causal inference attention (no autograd) returned as the output projection's input rows
    [B, Sq, Hq * D], which the kernel writes in place (no transpose copy); None when the call is not
    served by the library (the caller then takes its usual path). ``key_bits``/``window`` as in
    ``flash_forward``."""
    if not _GUARD.use_native(None, q, k, v):
        return None
    try:
        out = flash_forward(q, k, v, scale, True, num_kv_groups, causal_offset, need_lse=False, seq_major=True,
                            key_bits=key_bits, window=window)[0]
    except Exception as exc:
        _GUARD.failed(exc)
        return None
    return out.transpose(1, 2).reshape(q.shape[0], q.shape[2], -1)


def masked_attention(q, k, v, scale: float, num_kv_groups: int, causal_offset: int,
                     key_bits: torch.Tensor | None, window: int) -> torch.Tensor | None:
    """Causal inference attention with key padding and/or a sliding window ([B, Hq, Sq, D]); None
    when the call is not served by the library (autograd, fp32, CPU: the caller then applies the
    dense mask)."""
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        return None
    if q.dtype == torch.float32 or not _GUARD.use_native(None, q, k, v):
        return None
    try:
        return flash_forward(q, k, v, scale, True, num_kv_groups, causal_offset, need_lse=False,
                             key_bits=key_bits, window=window)[0]
    except Exception as exc:
        _GUARD.failed(exc)
        return None


def flash_backward(q, k, v, out, grad_out, lse, scale: float, causal: bool, num_kv_groups: int,
                   causal_offset: int = 0):
    q, k, v = _unit_last(q), _unit_last(k), _unit_last(v)
    B, Hq, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    o = out.contiguous()
    do = grad_out.to(q.dtype).contiguous()
    dq = torch.empty((B, Hq, Sq, D), dtype=q.dtype, device=q.device)
    dk = torch.empty((B, Hkv, Sk, D), dtype=k.dtype, device=k.device)
    dv = torch.empty((B, Hkv, Sk, D), dtype=v.dtype, device=v.device)
    ws = _native.workspace(_native.call("qh_flash_bwd_workspace", B, Hq, Sq), q.device)
    _native.call("qh_flash_bwd", q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(), k.stride(0),
                 k.stride(1), k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), o.data_ptr(),
                 do.data_ptr(), lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws.numel(),
                 B, Hq, Hkv, Sq, Sk, D, float(scale), int(bool(causal)), int(causal_offset),
                 _native.dtype_code(q.dtype), _native.stream(q.device))
    return dq, dk, dv


def flash_decode(q, k, v, scale: float, num_kv_groups: int, seqlens: torch.Tensor | None = None,
                 workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Single-query attention over all (or the first ``seqlens[b]``) keys; q [B,Hq,1,D]."""
    _check(q, k, v, num_kv_groups)
    if q.shape[2] != 1:
        raise Unsupported("flash_decode expects one query per sequence")
    k, v = _unit_last(k), _unit_last(v)
    q = _unit_last(q)
    B, Hq, _, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    out = torch.empty((B, Hq, 1, D), dtype=q.dtype, device=q.device)
    need = _native.call("qh_flash_decode_workspace", B, Hq, Hkv, Sk, D)
    if workspace is None or workspace.numel() < need:
        workspace = _native.workspace(need, q.device)
    if seqlens is not None and seqlens.dtype != torch.int32:
        raise Unsupported("seqlens must be int32")
    _native.call("qh_flash_decode", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
                 k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), out.data_ptr(), None,
                 None if seqlens is None else seqlens.data_ptr(), workspace.data_ptr(), workspace.numel(), B, Hq, Hkv,
                 Sk, D, float(scale), _native.dtype_code(q.dtype), _native.stream(q.device))
    return out


class _FlashAttentionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, scale, is_causal, num_kv_groups, causal_offset=0):
        out, lse = flash_forward(q, k, v, scale, is_causal, num_kv_groups, causal_offset)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.scale = scale
        ctx.is_causal = is_causal
        ctx.num_kv_groups = num_kv_groups
        ctx.causal_offset = causal_offset
        return out

    @staticmethod
    def backward(ctx, grad_output):
        q, k, v, out, lse = ctx.saved_tensors
        try:
            dq, dk, dv = flash_backward(q, k, v, out, grad_output, lse, ctx.scale, ctx.is_causal, ctx.num_kv_groups,
                                        ctx.causal_offset)
        except Exception as exc:
            _GUARD.failed(exc, "backward kernel")
            with torch.enable_grad():
                qq, kk, vv = (t.detach().requires_grad_(True) for t in (q, k, v))
                ref = _torch_attention_offset(qq, kk, vv, ctx.scale, ctx.is_causal, ctx.num_kv_groups,
                                              ctx.causal_offset)
                dq, dk, dv = torch.autograd.grad(ref, (qq, kk, vv), grad_output)
        return dq, dk, dv, None, None, None, None


def attention(q, k, v, scale: float, causal: bool, num_kv_groups: int, causal_offset: int = 0) -> torch.Tensor:
    """Dispatch used by the model layer: decode kernel for one query without grad, else flash fwd(/bwd)."""
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        return _FlashAttentionFunction.apply(q, k, v, scale, causal, num_kv_groups, causal_offset)
    if q.shape[2] == 1 and (not causal or causal_offset >= k.shape[2] - 1) and q.dtype != torch.float32:
        return flash_decode(q, k, v, scale, num_kv_groups)  # (fp32 single queries take the forward kernel)
    return flash_forward(q, k, v, scale, causal, num_kv_groups, causal_offset, need_lse=False)[0]


def triton_flash_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    is_causal: bool = True,
    num_kv_groups: int = 1,
    use_triton: bool | None = None,
) -> torch.Tensor:
    if not _GUARD.use_native(use_triton, q, k, v):
        return _torch_flash_attention(q, k, v, scale, is_causal, num_kv_groups)
    try:
        return attention(q, k, v, scale, is_causal, num_kv_groups, 0)
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_flash_attention(q, k, v, scale, is_causal, num_kv_groups)
