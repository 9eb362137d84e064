"""Per-layer KV cache with write-by-position (reference: qwen_triton/modules/cache.py:11-117).

Same fields and growth policy as the reference (power-of-two capacity, at least
16, capped by ``max_cache_len``; the view handed back is ``[:, :, :valid_len]``).
Additions: ``update_attention`` accepts ``max_position`` so callers that know the
largest written position on the host skip the ``positions.max().item()``
synchronisation, and ``reserve`` preallocates a layer's storage up front (no
regrowth copies during decoding). A layer's key and value storages are two views
of one buffer with their rows interleaved (``[B, H, cap, 2, D]``): a decode step
then streams one contiguous region per (sequence, kv-head) instead of two.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from qwen_triton.kernels import append_attention_kv, write_attention_kv


@dataclass
class StaticDecode:
    """Device-side state of a decode step that is captured once and replayed (HIP graph).

    ``positions`` (int64 [1]) is the cache position the step writes; ``seqlens`` (int32 [B]) is
    each sequence's valid key count after that write. The captured step reads both from device
    memory and advances them itself, so every replay decodes the next position without the host.
    """
    positions: torch.Tensor
    seqlens: torch.Tensor


@dataclass
class QwenTritonCache:
    num_layers: int
    layer_types: list[str]
    max_cache_len: int | None = None

    def __post_init__(self) -> None:
        self.key_cache: list[torch.Tensor | None] = [None] * self.num_layers
        self.value_cache: list[torch.Tensor | None] = [None] * self.num_layers
        self.conv_states: list[torch.Tensor | None] = [None] * self.num_layers
        self.recurrent_states: list[torch.Tensor | None] = [None] * self.num_layers
        self.attention_lengths: list[int] = [0] * self.num_layers
        # set by a graph-captured decode loop (see StaticDecode); None for ordinary use
        self.static: StaticDecode | None = None

    def _resolve_capacity(self, required_len: int) -> int:
        if required_len <= 0:
            return 16
        if self.max_cache_len is not None and required_len > self.max_cache_len:
            raise ValueError(f"Requested cache length {required_len} exceeds max_cache_len={self.max_cache_len}")
        capacity = max(16, 1 << (required_len - 1).bit_length())
        if self.max_cache_len is not None:
            capacity = min(capacity, self.max_cache_len)
        return max(required_len, capacity)

    @staticmethod
    def _compatible(storage: torch.Tensor | None, like: torch.Tensor) -> bool:
        return (
            storage is not None
            and storage.device == like.device
            and storage.dtype == like.dtype
            and storage.shape[0] == like.shape[0]
            and storage.shape[1] == like.shape[1]
            and storage.shape[3] == like.shape[3]
        )

    @staticmethod
    def _new_kv_pair(shape: tuple[int, int, int, int], dtype: torch.dtype,
                     device: torch.device | str) -> tuple[torch.Tensor, torch.Tensor]:
        """Key and value storage ``shape`` = (B, H, cap, D) as views of one [B, H, cap, 2, D] buffer."""
        b, h, cap, d = shape
        buf = torch.empty((b, h, cap, 2, d), dtype=dtype, device=device)
        return buf[:, :, :, 0, :], buf[:, :, :, 1, :]

    def _ensure_kv_storage(self, layer_idx: int, like_k: torch.Tensor, like_v: torch.Tensor, current_length: int,
                           required_len: int) -> None:
        """Grow a layer's key/value storages together (the reference grows each as
        ``_ensure_attention_storage`` does: power-of-two capacity, valid rows copied)."""
        k, v = self.key_cache[layer_idx], self.value_cache[layer_idx]
        if (self._compatible(k, like_k) and self._compatible(v, like_v) and k.shape[2] >= required_len
                and v.shape[2] >= required_len):
            return
        if like_k.shape[3] != like_v.shape[3] or like_k.dtype != like_v.dtype or like_k.shape[:2] != like_v.shape[:2]:
            self.key_cache[layer_idx] = self._ensure_attention_storage(k, like_k, current_length, required_len)
            self.value_cache[layer_idx] = self._ensure_attention_storage(v, like_v, current_length, required_len)
            return
        capacity = self._resolve_capacity(required_len)
        nk, nv = self._new_kv_pair((like_k.shape[0], like_k.shape[1], capacity, like_k.shape[3]), like_k.dtype,
                                   like_k.device)
        for old, new, like in ((k, nk, like_k), (v, nv, like_v)):
            if self._compatible(old, like) and current_length > 0:
                n = min(current_length, old.shape[2], capacity)
                new[:, :, :n].copy_(old[:, :, :n])
        self.key_cache[layer_idx], self.value_cache[layer_idx] = nk, nv

    def _ensure_attention_storage(self, storage, like, current_length: int, required_len: int) -> torch.Tensor:
        if self._compatible(storage, like) and storage.shape[2] >= required_len:
            return storage
        capacity = self._resolve_capacity(required_len)
        new_storage = like.new_empty((like.shape[0], like.shape[1], capacity, like.shape[3]))
        if self._compatible(storage, like) and current_length > 0:
            n = min(current_length, storage.shape[2], capacity)
            new_storage[:, :, :n].copy_(storage[:, :, :n])
        return new_storage

    def reserve(self, layer_idx: int, batch: int, heads: int, capacity: int, head_dim: int, dtype: torch.dtype,
                device: torch.device | str) -> None:
        """Preallocate key/value storage of ``capacity`` positions for one layer."""
        shape = (batch, heads, capacity, head_dim)
        cur_k, cur_v = self.key_cache[layer_idx], self.value_cache[layer_idx]
        if all(cur is not None and cur.shape[2] >= capacity and tuple(cur.shape[:2]) == shape[:2]
               and cur.shape[3] == head_dim for cur in (cur_k, cur_v)):
            return
        new_k, new_v = self._new_kv_pair(shape, dtype, device)
        n = self.attention_lengths[layer_idx]
        for cur, new in ((cur_k, new_k), (cur_v, new_v)):
            if cur is not None and n > 0 and tuple(cur.shape[:2]) == shape[:2] and cur.shape[3] == head_dim:
                new[:, :, :n].copy_(cur[:, :, :n])
        self.key_cache[layer_idx], self.value_cache[layer_idx] = new_k, new_v

    def update_attention(
        self,
        layer_idx: int,
        key_states: torch.Tensor,
        value_states: torch.Tensor,
        cache_position: torch.LongTensor | None = None,
        max_position: int | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        if cache_position is None:
            self.key_cache[layer_idx] = append_attention_kv(self.key_cache[layer_idx], key_states)
            self.value_cache[layer_idx] = append_attention_kv(self.value_cache[layer_idx], value_states)
            self.attention_lengths[layer_idx] = int(self.key_cache[layer_idx].shape[-2])
            return self.key_cache[layer_idx], self.value_cache[layer_idx]

        positions = cache_position.to(device=key_states.device, dtype=torch.long).reshape(-1)
        if positions.numel() != key_states.shape[-2]:
            raise ValueError("cache_position length must match the sequence dimension of key/value states")
        current = self.attention_lengths[layer_idx]
        if positions.numel() == 0:
            required = current
        elif max_position is not None:
            required = int(max_position) + 1
        else:
            required = int(positions.max().item()) + 1
        self._ensure_kv_storage(layer_idx, key_states, value_states, current, required)
        write_attention_kv(self.key_cache[layer_idx], key_states, positions)
        write_attention_kv(self.value_cache[layer_idx], value_states, positions)
        self.attention_lengths[layer_idx] = max(current, required)
        n = self.attention_lengths[layer_idx]
        return self.key_cache[layer_idx][:, :, :n, :], self.value_cache[layer_idx][:, :, :n, :]

    def claim_positions(self, layer_idx: int, batch: int, heads: int, head_dim: int, dtype: torch.dtype,
                        device: torch.device, positions: torch.Tensor,
                        max_position: int | None = None) -> tuple[torch.Tensor, torch.Tensor, int]:
        """Make room for writes at ``positions`` (as ``update_attention`` would) without writing.

        Returns the key/value storages and the new valid length; a fused kernel then
        writes the rows itself.
        """
        current = self.attention_lengths[layer_idx]
        if positions.numel() == 0:
            required = current
        elif max_position is not None:
            required = int(max_position) + 1
        else:
            required = int(positions.max().item()) + 1
        like = torch.empty((batch, heads, 0, head_dim), dtype=dtype, device=device)
        self._ensure_kv_storage(layer_idx, like, like, current, required)
        self.attention_lengths[layer_idx] = max(current, required)
        return self.key_cache[layer_idx], self.value_cache[layer_idx], self.attention_lengths[layer_idx]

    def capacity(self) -> int:
        """Reserved positions of the attention layers (0 if none is allocated)."""
        for key in self.key_cache:
            if key is not None:
                return key.shape[2]
        return 0

    def get_seq_length(self, layer_idx: int | None = None) -> int:
        if layer_idx is not None and self.key_cache[layer_idx] is not None:
            return self.attention_lengths[layer_idx]
        for idx, key in enumerate(self.key_cache):
            if key is not None:
                return self.attention_lengths[idx]
        return 0

    @property
    def has_previous_state(self) -> bool:
        linear = [i for i, t in enumerate(self.layer_types) if t == "linear_attention"]
        return bool(linear) and self.recurrent_states[linear[-1]] is not None
