"""Full (softmax) attention block (reference: qwen_triton/modules/attention.py:17-128).

Projections, per-head QK RMSNorm, RoPE, cache update and attention, with the
reference's parameter names. Dispatch differs from the reference on purpose
(its K1 defect: the model always passes a mask, so prefill never reached the
flash kernel):

* no mask: causal flash attention, aligned bottom-right when queries sit on
  top of cached keys (``causal_offset = kv_len - q_len``); a single query takes
  the split-KV decode kernel;
* padding and/or sliding-window mask (``CausalPaddingMask``): the masked flash
  kernel for inference in bf16/fp16 on the GPU; otherwise (autograd, fp32, CPU)
  the additive mask with fp32 SDPA over repeated KV heads, as the reference does
  for masked multi-token attention;
* explicit additive mask tensor: that fp32 SDPA.

Inference (no autograd, GPU, position-indexed cache): the q/k/v projections
of up to 128 tokens run as one grouped launch, and q_norm/k_norm, RoPE and the
cache writes as one fused pass (``qh_attn_prepare``), both with the same
arithmetic as the separate kernels.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from qwen_triton import _native
from qwen_triton.configs import QwenTritonConfig
from qwen_triton.kernels import sigmoid_mul
from qwen_triton.kernels import flash_attention as _fa
from qwen_triton.kernels.flash_attention import triton_flash_attention
from qwen_triton.kernels.matmul import linear_group, linear_group_ok
from qwen_triton.modules.cache import QwenTritonCache
from qwen_triton.modules.linear import TritonLinear
from qwen_triton.modules.norms import QwenRMSNorm
from qwen_triton.modules.rotary import apply_rotary_pos_emb


# Decode steps (one new token per sequence) of many sequences run the q/k norm, RoPE and cache
# writes inside the decode-attention kernel (``qh_flash_decode_prepare``); False keeps the
# separate prepare pass. Both give identical results.
FUSE_DECODE_PREPARE = True


def repeat_kv(hidden_states: torch.Tensor, n_rep: int) -> torch.Tensor:
    b, h, s, d = hidden_states.shape
    if n_rep == 1:
        return hidden_states
    return hidden_states[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


class CausalPaddingMask:
    """The decoder's causal mask (optionally a sliding window) with key padding, kept in the
    structured form the masked flash kernel applies; the reference builds it as an additive fp32
    [B, 1, q, kv] tensor (qwen_triton/models/core.py:47-75) that every layer then reads.

    Query i of the step sits at cache position ``past + i`` and sees key j < kv_len iff
    j <= past + i, j > past + i - window (when a window is set) and ``key_valid[b, j]`` is
    non-zero. ``dense()`` builds the additive tensor once, for the calls the kernel does not take
    (autograd, fp32, CPU, caller-given cache positions)."""

    def __init__(self, build_dense, key_valid: torch.Tensor | None, past: int, q_len: int,
                 window: int | None, positions_known: bool) -> None:
        self._build_dense = build_dense
        self._dense: torch.Tensor | None = None
        self._bits: torch.Tensor | None = None
        self.key_valid = key_valid  # [B, kv_len] or None
        self.past, self.q_len, self.kv_len = past, q_len, past + q_len
        self.window = window
        self.positions_known = positions_known  # the step's cache positions are past .. past + q_len - 1

    def dense(self) -> torch.Tensor:
        if self._dense is None:
            self._dense = self._build_dense()
        return self._dense

    def kernel_args(self, q: torch.Tensor, k: torch.Tensor):
        """(key_bits or None, window, causal_offset) for the masked kernel, or None when this call
        needs the dense mask."""
        if not self.positions_known or k.shape[2] != self.kv_len or q.shape[2] != self.q_len:
            return None
        if self.window is not None and self.window <= 0:
            return None
        if self.key_valid is not None:
            if self.key_valid.shape[0] != q.shape[0]:
                return None
            if self._bits is None:
                self._bits = _fa.pack_key_bits(self.key_valid.to(q.device))
        return self._bits, self.window or 0, self.past


class QwenFullAttention(nn.Module):
    def __init__(self, config: QwenTritonConfig, layer_idx: int) -> None:
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.head_dim = config.head_dim
        self.num_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        self.num_key_value_groups = config.num_attention_heads // config.num_key_value_heads
        self.scaling = self.head_dim ** -0.5
        self.attention_dropout = config.attention_dropout
        q_out = config.num_attention_heads * self.head_dim * (2 if config.attn_output_gate else 1)
        kv_out = config.num_key_value_heads * self.head_dim
        self.q_proj = TritonLinear(config.hidden_size, q_out, bias=config.attention_bias)
        self.k_proj = TritonLinear(config.hidden_size, kv_out, bias=config.attention_bias)
        self.v_proj = TritonLinear(config.hidden_size, kv_out, bias=config.attention_bias)
        self.o_proj = TritonLinear(config.num_attention_heads * self.head_dim, config.hidden_size,
                                   bias=config.attention_bias)
        self.q_norm = QwenRMSNorm(self.head_dim, eps=config.rms_norm_eps, one_plus_weight=config.norm_one_plus)
        self.k_norm = QwenRMSNorm(self.head_dim, eps=config.rms_norm_eps, one_plus_weight=config.norm_one_plus)

    def _attend(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                mask: torch.Tensor | CausalPaddingMask | None, out_dtype: torch.dtype) -> torch.Tensor:
        q_len, kv_len = q.shape[2], k.shape[2]
        groups = self.num_key_value_groups
        if isinstance(mask, CausalPaddingMask):
            args = mask.kernel_args(q, k)
            if args is not None:
                out = _fa.masked_attention(q, k, v, self.scaling, groups, args[2], args[0], args[1])
                if out is not None:
                    return out.to(out_dtype)
            mask = mask.dense()
        if mask is None:
            on_gpu = q.is_cuda and k.is_cuda
            if on_gpu:
                if q_len == kv_len:
                    return triton_flash_attention(q, k, v, scale=self.scaling, is_causal=True, num_kv_groups=groups)
                return _fa.attention(q, k, v, self.scaling, True, groups, causal_offset=kv_len - q_len)
            # CPU: reference torch semantics, bottom-right causal.
            if q_len == kv_len:
                return _fa._torch_flash_attention(q, k, v, self.scaling, True, groups)
            if q_len == 1:
                return _fa._torch_flash_attention(q, k, v, self.scaling, False, groups)
            pos_q = torch.arange(kv_len - q_len, kv_len, device=q.device)
            allowed = torch.arange(kv_len, device=q.device)[None, :] <= pos_q[:, None]
            mask = torch.zeros((q_len, kv_len), device=q.device, dtype=torch.float32).masked_fill(
                ~allowed, torch.finfo(torch.float32).min)[None, None]
        ke, ve = repeat_kv(k, groups), repeat_kv(v, groups)
        m = mask[:, :, :, :kv_len]
        return torch.nn.functional.scaled_dot_product_attention(
            q.to(torch.float32), ke.to(torch.float32), ve.to(torch.float32), attn_mask=m, dropout_p=0.0,
            is_causal=False, scale=self.scaling).to(out_dtype)

    def _fused_prepare_ok(self, hidden_states: torch.Tensor, cos: torch.Tensor, past_key_values,
                          cache_position) -> bool:
        d, rot = self.head_dim, cos.shape[-1]
        half_lanes = rot // 16
        return (not torch.is_grad_enabled() and hidden_states.is_cuda and hidden_states.dim() == 3
                and hidden_states.dtype in (torch.bfloat16, torch.float16) and not self.config.attn_output_gate
                and past_key_values is not None and cache_position is not None
                and d % 8 == 0 and d <= 128 and rot % 16 == 0 and 16 <= rot <= d
                and half_lanes & (half_lanes - 1) == 0
                and cos.dim() == 3 and cos.shape[0] in (1, hidden_states.shape[0])
                and cos.shape[1] == hidden_states.shape[1] and cos.dtype in (torch.float32, hidden_states.dtype)
                and self.q_norm.weight.dtype in (torch.float32, hidden_states.dtype)
                and self.k_norm.weight.dtype == self.q_norm.weight.dtype
                and _native.available())

    def _fused_prepare(self, q2: torch.Tensor, k2: torch.Tensor, v2: torch.Tensor, cos: torch.Tensor,
                       sin: torch.Tensor, past_key_values: QwenTritonCache, cache_position: torch.Tensor,
                       max_position: int | None):
        """q_norm/k_norm + RoPE + cache write in one launch; returns q [B,Hq,S,D] and the cache views."""
        bsz, seq = q2.shape[0], q2.shape[1]
        hq, hkv, d = self.num_heads, self.num_key_value_heads, self.head_dim
        positions = cache_position.to(device=q2.device, dtype=torch.long).reshape(-1)
        if positions.numel() != seq:
            raise ValueError("cache_position length must match the sequence dimension of key/value states")
        kc, vc, n = past_key_values.claim_positions(self.layer_idx, bsz, hkv, d, q2.dtype, q2.device, positions,
                                                    max_position)
        q2, k2, v2 = (t.reshape(bsz * seq, -1) for t in (q2, k2, v2))
        if q2.stride(1) != 1 or k2.stride(1) != 1 or v2.stride(1) != 1:
            q2, k2, v2 = q2.contiguous(), k2.contiguous(), v2.contiguous()
        if cos.stride(-1) != 1 or sin.stride() != cos.stride():
            cos, sin = cos.contiguous(), sin.contiguous()
        q_out = torch.empty((bsz, hq, seq, d), dtype=q2.dtype, device=q2.device)
        wq, wk = self.q_norm.weight, self.k_norm.weight
        _native.call("qh_attn_prepare", q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0), v2.data_ptr(),
                     v2.stride(0), wq.data_ptr(), wk.data_ptr(), float(self.q_norm.eps),
                     int(self.q_norm.one_plus_weight), cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.stride(1),
                     cos.shape[0], cos.shape[-1], q_out.data_ptr(), kc.data_ptr(), *kc.stride()[:3], vc.data_ptr(),
                     *vc.stride()[:3], positions.data_ptr(), bsz, seq, hq, hkv, d, kc.shape[2],
                     _native.dtype_code(q2.dtype), _native.dtype_code(wq.dtype), _native.dtype_code(cos.dtype),
                     _native.stream(q2.device))
        return q_out, kc[:, :, :n, :], vc[:, :, :n, :]

    def _decode_prepare_ok(self, q2: torch.Tensor, attention_mask, cos: torch.Tensor, sin: torch.Tensor) -> bool:
        # cos/sin in the activation dtype: the fused kernel's products are then all exact in fp32
        # and its rows equal the prepare pass's bit for bit
        if not (FUSE_DECODE_PREPARE and attention_mask is None and q2.shape[1] == 1 and cos.shape[1] == 1
                and sin.shape == cos.shape and cos.dtype == q2.dtype and sin.dtype == q2.dtype
                and cos.data_ptr() % 16 == 0 and sin.data_ptr() % 16 == 0 and cos.stride(0) % 8 == 0
                and cos.stride(-1) == 1 and sin.stride() == cos.stride()
                and self.q_norm.weight.data_ptr() % 16 == 0 and self.k_norm.weight.data_ptr() % 16 == 0
                and self.k_norm.weight.dtype == self.q_norm.weight.dtype
                and self.q_norm.weight.dtype in (torch.float32, q2.dtype)):
            return False
        return True

    def _fused_decode(self, q2: torch.Tensor, k2: torch.Tensor, v2: torch.Tensor, cos: torch.Tensor,
                      sin: torch.Tensor, past_key_values: QwenTritonCache, cache_position: torch.Tensor,
                      max_position: int | None) -> torch.Tensor:
        """One decode step (a token per sequence): q/k norm, RoPE, the cache writes and the attention
        in one launch; returns ``[B, Hq, D]``, or None (nothing launched) for shapes the kernel does
        not serve."""
        bsz = q2.shape[0]
        hq, hkv, d = self.num_heads, self.num_key_value_heads, self.head_dim
        positions = cache_position.to(device=q2.device, dtype=torch.long).reshape(-1)
        if positions.numel() != 1:
            raise ValueError("cache_position length must match the sequence dimension of key/value states")
        kc, vc, n = past_key_values.claim_positions(self.layer_idx, bsz, hkv, d, q2.dtype, q2.device, positions,
                                                    max_position)
        static = getattr(past_key_values, "static", None)
        # captured decode step: keys span the reserved cache, each sequence's valid length is read
        # from device memory
        seqlens, sk = (static.seqlens, kc.shape[2]) if static is not None else (None, n)
        # many sequences, or few keys (the kernel's own rule); otherwise the caller takes the
        # prepare pass and the split decode kernel
        if not _native.call("qh_flash_decode_prepare_ok", bsz, hq, hkv, sk, d):
            return None
        q2, k2, v2 = (t.reshape(bsz, -1) for t in (q2, k2, v2))
        if q2.stride(1) != 1 or k2.stride(1) != 1 or v2.stride(1) != 1:
            q2, k2, v2 = q2.contiguous(), k2.contiguous(), v2.contiguous()
        if cos.stride(-1) != 1 or sin.stride() != cos.stride():
            cos, sin = cos.contiguous(), sin.contiguous()
        out = torch.empty((bsz, hq, d), dtype=q2.dtype, device=q2.device)
        wq, wk = self.q_norm.weight, self.k_norm.weight
        _native.call("qh_flash_decode_prepare", q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0),
                     v2.data_ptr(), v2.stride(0), wq.data_ptr(), wk.data_ptr(), float(self.q_norm.eps),
                     int(self.q_norm.one_plus_weight), cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0],
                     cos.shape[-1], kc.data_ptr(), *kc.stride()[:3], vc.data_ptr(), *vc.stride()[:3], kc.shape[2],
                     positions.data_ptr(), out.data_ptr(), None, None if seqlens is None else seqlens.data_ptr(),
                     bsz, hq, hkv, sk, d, float(self.scaling), _native.dtype_code(q2.dtype),
                     _native.dtype_code(wq.dtype), _native.dtype_code(cos.dtype), _native.stream(q2.device))
        return out

    def attend_projected(self, q2: torch.Tensor, k2: torch.Tensor, v2: torch.Tensor,
                         position_embeddings: tuple[torch.Tensor, torch.Tensor], attention_mask, past_key_values,
                         cache_position, max_position: int | None) -> torch.Tensor:
        """Inference after the projections (``_fused_prepare_ok`` holds): q/k norm, RoPE and cache
        write in one pass, then attention; returns the o_proj input ``[B, S, Hq * D]``."""
        cos, sin = position_embeddings
        input_shape = q2.shape[:-1]
        if self._decode_prepare_ok(q2, attention_mask, cos, sin):
            out = self._fused_decode(q2, k2, v2, cos, sin, past_key_values, cache_position, max_position)
            if out is not None:
                return out.view(*input_shape, -1)
        q, k, v = self._fused_prepare(q2, k2, v2, cos, sin, past_key_values, cache_position, max_position)
        static = getattr(past_key_values, "static", None)
        if static is not None and q.shape[2] == 1 and attention_mask is None:
            # captured decode step: k/v span the reserved cache, each sequence's valid length
            # is read from device memory
            out = _fa.flash_decode(q, k, v, self.scaling, self.num_key_value_groups, seqlens=static.seqlens)
        else:
            if attention_mask is None and q.shape[2] > 1:
                rows = _fa.attention_rows(q, k, v, self.scaling, self.num_key_value_groups,
                                          causal_offset=k.shape[2] - q.shape[2])
                if rows is not None:
                    return rows.view(*input_shape, -1)
            if isinstance(attention_mask, CausalPaddingMask) and q.shape[2] > 1:
                args = attention_mask.kernel_args(q, k)
                if args is not None:
                    rows = _fa.attention_rows(q, k, v, self.scaling, self.num_key_value_groups,
                                              causal_offset=args[2], key_bits=args[0], window=args[1])
                    if rows is not None:
                        return rows.view(*input_shape, -1)
            out = self._attend(q, k, v, attention_mask, q2.dtype)
        return out.transpose(1, 2).reshape(*input_shape, -1)

    def forward(
        self,
        hidden_states: torch.Tensor,
        position_embeddings: tuple[torch.Tensor, torch.Tensor],
        attention_mask: Optional[torch.Tensor] = None,
        past_key_values: Optional[QwenTritonCache] = None,
        cache_position: Optional[torch.LongTensor] = None,
        max_position: int | None = None,
    ) -> torch.Tensor:
        input_shape = hidden_states.shape[:-1]
        cos, sin = position_embeddings
        if self._fused_prepare_ok(hidden_states, cos, past_key_values, cache_position):
            projs = (self.q_proj, self.k_proj, self.v_proj)
            weights = [p.weight for p in projs]
            if linear_group_ok(hidden_states, weights):
                q2, k2, v2 = linear_group(hidden_states, weights, [p.bias for p in projs])
            else:
                q2, k2, v2 = (p(hidden_states) for p in projs)
            out = self.attend_projected(q2, k2, v2, position_embeddings, attention_mask, past_key_values,
                                        cache_position, max_position)
            return self.o_proj(out)
        if getattr(past_key_values, "static", None) is not None:
            raise RuntimeError("a captured decode step needs the fused inference path (bf16/fp16 on the GPU, "
                               "no output gate, no autograd)")
        mixed_q = self.q_proj(hidden_states)
        gate = None
        if self.config.attn_output_gate:
            q, gate = torch.chunk(mixed_q.view(*input_shape, -1, self.head_dim * 2), 2, dim=-1)
            gate = gate.reshape(*input_shape, -1)
        else:
            q = mixed_q.view(*input_shape, -1, self.head_dim)
        k = self.k_proj(hidden_states).view(*input_shape, -1, self.head_dim)
        v = self.v_proj(hidden_states).view(*input_shape, -1, self.head_dim)

        q = self.q_norm(q).transpose(1, 2)
        k = self.k_norm(k).transpose(1, 2)
        v = v.transpose(1, 2)
        q, k = apply_rotary_pos_emb(q, k, cos, sin)

        if past_key_values is not None:
            k, v = past_key_values.update_attention(self.layer_idx, k, v, cache_position=cache_position,
                                                    max_position=max_position)
        out = self._attend(q, k, v, attention_mask, hidden_states.dtype)
        out = out.transpose(1, 2).reshape(*input_shape, -1)
        if gate is not None:
            out = sigmoid_mul(out, gate)
        return self.o_proj(out)
