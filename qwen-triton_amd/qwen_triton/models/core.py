"""Qwen3 / Qwen3-MoE causal LM on the MI355X operator stack.

Reference: qwen_triton/models/core.py:1-409 (mask builder :47-74, loss shift
:85-92, decoder layer :95-153, model :156-247, causal LM + greedy decode
:250-409). Public API, parameter names and output types are the reference's.
Differences, all in the dispatch rather than the maths:

* without a padding mask the layers get ``attention_mask=None`` and run causal
  flash attention (the reference always built an additive mask, which sent
  every prefill to fp32 SDPA); with one, or with a sliding window, they get a
  ``CausalPaddingMask``, which inference in bf16/fp16 applies inside the flash
  kernel and every other call as the reference's additive tensor;
* the largest cache position is known on the host when ``cache_position`` is
  generated here, so the cache write needs no device-to-host sync;
* ``greedy_generate`` preallocates the KV cache for the whole generation;
* inference with at most 128 tokens runs each dense layer as five launches: the
  input norm inside the q/k/v product, the attention, o_proj with the residual
  add, the post-attention norm inside the gate/up product, down_proj with the
  residual add (``FUSE_NORM_GEMM``; a fused norm rounds the operand
  ``x * weight`` and applies the row factor after the product, where the RMSNorm
  kernel rounds ``x * factor * weight``: one rounding step placed differently).
"""
from __future__ import annotations

from types import SimpleNamespace
from typing import Any

import torch
from torch import nn
from transformers.modeling_outputs import CausalLMOutputWithPast

from qwen_triton.configs import QwenTritonConfig
from qwen_triton.kernels.cross_entropy import triton_cross_entropy
from qwen_triton.kernels import matmul as _matmul
from qwen_triton.kernels.matmul import linear_group, linear_group_norm_ok, linear_group_ok
from qwen_triton.kernels.residual_add import residual_add
from qwen_triton.kernels.rmsnorm import add_rmsnorm, add_rmsnorm_ok
from qwen_triton.modules import (
    Qwen3NextLinearAttention,
    QwenFullAttention,
    QwenMLP,
    QwenRMSNorm,
    QwenRotaryEmbedding,
    QwenSparseMoeBlock,
    QwenTritonCache,
)
from qwen_triton.modules.attention import CausalPaddingMask
from qwen_triton.modules.cache import StaticDecode
from qwen_triton.modules.embedding import TritonEmbedding
from qwen_triton.modules.linear import TritonLinear

# Inference on the GPU with at most 128 tokens: fold each dense layer's norms and residual
# adds into its projections (see QwenDecoderLayer.forward_fused). False keeps the separate
# (bitwise-reference) kernels.
FUSE_NORM_GEMM = True

_DTYPES = {
    "fp16": torch.float16, "float16": torch.float16, "half": torch.float16,
    "bf16": torch.bfloat16, "bfloat16": torch.bfloat16,
    "fp32": torch.float32, "float32": torch.float32,
}


def _parse_dtype(dtype: torch.dtype | str | None) -> torch.dtype | None:
    if dtype is None or isinstance(dtype, torch.dtype):
        return dtype
    try:
        return _DTYPES[dtype.lower()]
    except KeyError:
        raise ValueError(f"Unsupported dtype string: {dtype}") from None


def _build_causal_mask(attention_mask, batch_size: int, cache_position, device, past: int, window_size=None):
    """Additive fp32 mask [B, 1, q, kv]: causal (optionally windowed) plus key padding; ``past`` is the
    number of cached keys before this step."""
    q_len = cache_position.shape[0]
    kv_len = past + q_len
    keys = torch.arange(kv_len, device=device)
    allowed = keys[None, :] <= cache_position[:, None]
    if window_size is not None:
        allowed = allowed & (keys[None, :] > cache_position[:, None] - window_size)
    neg = torch.finfo(torch.float32).min
    mask = torch.full((q_len, kv_len), neg, device=device, dtype=torch.float32).masked_fill(allowed, 0.0)
    mask = mask[None, None].expand(batch_size, 1, q_len, kv_len)
    if attention_mask is not None:
        am = attention_mask.to(device)
        if am.shape[1] < kv_len:
            am = torch.cat((torch.ones((am.shape[0], kv_len - am.shape[1]), device=device, dtype=am.dtype), am), dim=-1)
        mask = mask + (1.0 - am[:, None, None, :kv_len].to(torch.float32)) * neg
    return mask


def _structured_mask(attention_mask, batch_size: int, cache_position, device, past_key_values, window_size,
                     positions_known: bool) -> CausalPaddingMask:
    """``_build_causal_mask``'s mask in structured form: the key-validity rows it adds (ones
    prepended for cached keys the 2-D mask does not cover) and the window; the additive tensor is
    built only if a layer asks for it, with the cache length read here, before any layer of the
    step has appended its keys."""
    q_len = cache_position.shape[0]
    past = 0 if past_key_values is None else past_key_values.get_seq_length()
    kv_len = past + q_len
    key_valid = None
    if attention_mask is not None:
        am = attention_mask.to(device)
        if am.shape[1] < kv_len:
            am = torch.cat((torch.ones((am.shape[0], kv_len - am.shape[1]), device=device, dtype=am.dtype), am), dim=-1)
        key_valid = am[:, :kv_len]

    def build():
        return _build_causal_mask(attention_mask, batch_size, cache_position, device, past, window_size)

    return CausalPaddingMask(build, key_valid, past, q_len, window_size, positions_known)


def _layer_uses_moe(config: QwenTritonConfig, layer_idx: int) -> bool:
    if not config.is_moe or config.num_experts <= 0 or layer_idx in config.mlp_only_layers:
        return False
    return (layer_idx + 1) % config.decoder_sparse_step == 0


def _loss_fn(logits: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
    """Mean next-token cross-entropy (reference: qwen_triton/models/core.py, logits[:, :-1] against
    labels[:, 1:]). The labels are shifted instead of the logits: position s is scored against
    labels[:, s + 1] and each sequence's last position is ignored, so the logits enter as a
    [B * S, V] view (slicing them would copy the whole tensor for B > 1, and its gradient again)
    and the mean over the valid positions is the same."""
    if labels.shape != logits.shape[:-1]:
        raise ValueError(f"labels {tuple(labels.shape)} do not match logits {tuple(logits.shape)}")
    shift_labels = torch.full_like(labels, -100)
    shift_labels[:, :-1] = labels[:, 1:]
    return triton_cross_entropy(logits.reshape(-1, logits.shape[-1]), shift_labels.reshape(-1), ignore_index=-100)


class QwenDecoderLayer(nn.Module):
    def __init__(self, config: QwenTritonConfig, layer_idx: int) -> None:
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.layer_type = config.layer_types[layer_idx]
        eps, one_plus = config.rms_norm_eps, config.norm_one_plus
        self.input_layernorm = QwenRMSNorm(config.hidden_size, eps=eps, one_plus_weight=one_plus)
        self.post_attention_layernorm = QwenRMSNorm(config.hidden_size, eps=eps, one_plus_weight=one_plus)
        if self.layer_type == "linear_attention":
            self.linear_attn = Qwen3NextLinearAttention(config, layer_idx)
        else:
            self.self_attn = QwenFullAttention(config, layer_idx)
        self.mlp = QwenSparseMoeBlock(config) if _layer_uses_moe(config, layer_idx) else QwenMLP(
            config.hidden_size, config.intermediate_size)

    def _add_norm(self, x: torch.Tensor, residual: torch.Tensor, norm: QwenRMSNorm):
        """(x + residual, norm(x + residual)), fused into one pass for inference."""
        if add_rmsnorm_ok(x, residual, norm.weight):
            return add_rmsnorm(x, residual, norm.weight, norm.eps, norm.one_plus_weight)
        s = residual_add(x, residual)
        return s, norm(s)

    def fused_inference_ok(self, hidden_states: torch.Tensor, position_embeddings, past_key_values,
                           cache_position) -> bool:
        """Whether ``forward_fused`` serves this call: a full-attention layer with a dense MLP,
        inference on the GPU (bf16/fp16, at most 128 tokens, position-indexed cache), shapes the
        fused launches take."""
        if not FUSE_NORM_GEMM or torch.is_grad_enabled() or self.layer_type != "full_attention":
            return False
        if not isinstance(self.mlp, QwenMLP) or not hidden_states.is_cuda or hidden_states.dim() != 3:
            return False
        attn, mlp = self.self_attn, self.mlp
        if not attn._fused_prepare_ok(hidden_states, position_embeddings[0], past_key_values, cache_position):
            return False
        # the answer depends on the activation shape and on the weights (a cast or a reassignment
        # of the parameters changes their dtype or storage)
        key = (hidden_states.shape[0] * hidden_states.shape[1], hidden_states.dtype, hidden_states.device,
               _matmul.FOLD_NORM_WEIGHTS) + tuple(
            (w.data_ptr(), w.dtype) for w in (attn.q_proj.weight, attn.o_proj.weight, mlp.gate_proj.weight,
                                              mlp.down_proj.weight, self.input_layernorm.weight,
                                              self.post_attention_layernorm.weight))
        cache = self.__dict__.setdefault("_fused_ok_cache", {})
        if key not in cache:
            rows = hidden_states.reshape(-1, hidden_states.shape[-1])
            qkv = [attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight]
            gu = [mlp.gate_proj.weight, mlp.up_proj.weight]
            o_in = torch.empty((rows.shape[0], attn.o_proj.weight.shape[1]), dtype=rows.dtype, device=rows.device)
            d_in = torch.empty((rows.shape[0], mlp.down_proj.weight.shape[1]), dtype=rows.dtype, device=rows.device)
            cache[key] = (mlp.gate_proj.bias is None and mlp.up_proj.bias is None
                          and attn.o_proj.weight.shape[0] == rows.shape[1] == mlp.down_proj.weight.shape[0]
                          and linear_group_norm_ok(rows, qkv, self.input_layernorm.weight)
                          and linear_group_norm_ok(rows, gu, self.post_attention_layernorm.weight, gated=True)
                          and linear_group_ok(o_in, [attn.o_proj.weight])
                          and linear_group_ok(d_in, [mlp.down_proj.weight]))
        return cache[key]

    def forward_fused(self, hidden_states, position_embeddings, attention_mask=None, past_key_values=None,
                      cache_position=None, max_position: int | None = None) -> torch.Tensor:
        """The layer in five launches (``fused_inference_ok``); ``hidden_states`` is the full residual
        stream and so is the result."""
        attn, mlp = self.self_attn, self.mlp
        ln1, ln2 = self.input_layernorm, self.post_attention_layernorm
        projs = (attn.q_proj, attn.k_proj, attn.v_proj)
        q2, k2, v2 = linear_group(hidden_states, [p.weight for p in projs], [p.bias for p in projs],
                                  norm=(ln1.weight, ln1.eps, ln1.one_plus_weight))
        out = attn.attend_projected(q2, k2, v2, position_embeddings, attention_mask, past_key_values,
                                    cache_position, max_position)
        h = linear_group(out, [attn.o_proj.weight], [attn.o_proj.bias], residual=[hidden_states])[0]
        gu = linear_group(h, [mlp.gate_proj.weight, mlp.up_proj.weight], gated=True,
                          norm=(ln2.weight, ln2.eps, ln2.one_plus_weight))
        return linear_group(gu, [mlp.down_proj.weight], [mlp.down_proj.bias], residual=[h])[0]

    def forward(self, hidden_states, position_embeddings, attention_mask=None, past_key_values=None,
                cache_position=None, max_position: int | None = None, residual_in: torch.Tensor | None = None,
                defer_residual: bool = False):
        """Reference contract: returns ``(hidden_states, router_logits)``.

        For inference chains the model may pass ``residual_in`` (``hidden_states`` is then the
        previous layer's un-added output) and ``defer_residual`` (return ``(mlp_out,
        router_logits, residual)`` without the final add), so that each residual add is fused
        with the norm that follows it.
        """
        if residual_in is not None:
            residual, h = self._add_norm(hidden_states, residual_in, self.input_layernorm)
        else:
            residual = hidden_states
            h = self.input_layernorm(hidden_states)
        if self.layer_type == "linear_attention":
            h = self.linear_attn(hidden_states=h, cache_params=past_key_values, cache_position=cache_position,
                                 attention_mask=attention_mask)
        else:
            h = self.self_attn(hidden_states=h, position_embeddings=position_embeddings,
                               attention_mask=attention_mask, past_key_values=past_key_values,
                               cache_position=cache_position, max_position=max_position)
        residual, h = self._add_norm(h, residual, self.post_attention_layernorm)
        h = self.mlp(h)
        router_logits = None
        if isinstance(h, tuple):
            h, router_logits = h
        if defer_residual:
            return h, router_logits, residual
        return residual_add(h, residual), router_logits


class QwenTritonModel(nn.Module):
    def __init__(self, config: QwenTritonConfig) -> None:
        super().__init__()
        self.config = config
        self.embed_tokens = TritonEmbedding(config.vocab_size, config.hidden_size, config.pad_token_id)
        self.layers = nn.ModuleList([QwenDecoderLayer(config, i) for i in range(config.num_hidden_layers)])
        self.norm = QwenRMSNorm(config.hidden_size, eps=config.rms_norm_eps, one_plus_weight=config.norm_one_plus)
        self.rotary_emb = QwenRotaryEmbedding(config)

    @staticmethod
    def _mask_is_trivial(attention_mask: torch.Tensor | None) -> bool:
        return attention_mask is None or bool((attention_mask == 1).all())

    def forward(self, input_ids=None, attention_mask=None, position_ids=None, past_key_values=None, inputs_embeds=None,
                use_cache=None, cache_position=None, output_router_logits: bool = False, **_: Any):
        if (input_ids is None) == (inputs_embeds is None):
            raise ValueError("Specify exactly one of input_ids or inputs_embeds")
        if inputs_embeds is None:
            inputs_embeds = self.embed_tokens(input_ids)
        if use_cache and past_key_values is None:
            past_key_values = QwenTritonCache(self.config.num_hidden_layers, self.config.layer_types,
                                              max_cache_len=self.config.max_position_embeddings)
        seq = inputs_embeds.shape[1]
        max_position = None
        generated_positions = cache_position is None
        static = getattr(past_key_values, "static", None)
        if static is not None and cache_position is None:
            # captured decode step: the position lives in device memory; the attention reads
            # the whole reserved cache with per-sequence valid lengths
            cache_position = static.positions
            max_position = past_key_values.capacity() - 1
        elif cache_position is None:
            past = 0 if past_key_values is None else past_key_values.get_seq_length()
            cache_position = torch.arange(past, past + seq, device=inputs_embeds.device)
            max_position = past + seq - 1
        rope_bound = None
        if position_ids is None:
            position_ids = cache_position.unsqueeze(0)
            rope_bound = max_position  # every position id is at most max_position

        batch = inputs_embeds.shape[0]
        plain_causal = generated_positions and self._mask_is_trivial(attention_mask)
        # generated positions are past .. past + seq - 1 (a captured decode step's are not known)
        positions_known = generated_positions and static is None
        masks: dict[str, CausalPaddingMask | None] = {}
        if plain_causal:
            masks["full_attention"] = None
        else:
            masks["full_attention"] = _structured_mask(attention_mask, batch, cache_position, inputs_embeds.device,
                                                       past_key_values, None, positions_known)
        if "sliding_attention" in self.config.layer_types and self.config.sliding_window is not None:
            masks["sliding_attention"] = _structured_mask(attention_mask, batch, cache_position,
                                                          inputs_embeds.device, past_key_values,
                                                          self.config.sliding_window, positions_known)

        hidden = inputs_embeds
        position_embeddings = self.rotary_emb(hidden, position_ids, rope_bound)
        router_logits: list[torch.Tensor] = []
        # Inference on GPU: each layer's closing residual add is fused with the next norm.
        chain = add_rmsnorm_ok(hidden, hidden, self.norm.weight)
        residual = None
        for layer in self.layers:
            layer_mask = attention_mask if layer.layer_type == "linear_attention" else masks[layer.layer_type]
            if chain and layer.fused_inference_ok(hidden, position_embeddings, past_key_values, cache_position):
                if residual is not None:  # the previous layer deferred its closing add
                    hidden, residual = residual_add(hidden, residual), None
                hidden = layer.forward_fused(hidden, position_embeddings=position_embeddings,
                                             attention_mask=layer_mask, past_key_values=past_key_values,
                                             cache_position=cache_position, max_position=max_position)
                continue
            out = layer(hidden, position_embeddings=position_embeddings, attention_mask=layer_mask,
                        past_key_values=past_key_values, cache_position=cache_position, max_position=max_position,
                        residual_in=residual, defer_residual=chain)
            if chain:
                hidden, layer_router, residual = out
            else:
                hidden, layer_router = out
            if output_router_logits and layer_router is not None:
                router_logits.append(layer_router)
        if chain and residual is not None:
            if add_rmsnorm_ok(hidden, residual, self.norm.weight):
                _, hidden = add_rmsnorm(hidden, residual, self.norm.weight, self.norm.eps, self.norm.one_plus_weight)
            else:
                hidden = self.norm(residual_add(hidden, residual))
        else:
            hidden = self.norm(hidden)
        return SimpleNamespace(
            last_hidden_state=hidden,
            past_key_values=past_key_values if use_cache else None,
            router_logits=tuple(router_logits) if output_router_logits else None,
        )


class QwenTritonForCausalLM(nn.Module):
    def __init__(self, config: QwenTritonConfig, backend: str = "triton", init_weights: bool = True) -> None:
        super().__init__()
        if backend != "triton":
            raise ValueError("Use from_reference_model for backend='ref'")
        self.config = config
        self.backend = backend
        self.ref_model = None
        self.model = QwenTritonModel(config)
        self.lm_head = TritonLinear(config.hidden_size, config.vocab_size, bias=False)
        if init_weights:
            self._reset_parameters()
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    def _reset_parameters(self) -> None:
        std = self.config.initializer_range
        for module in self.modules():
            if isinstance(module, (nn.Linear, TritonLinear)):
                nn.init.normal_(module.weight, mean=0.0, std=std)
                if module.bias is not None:
                    nn.init.zeros_(module.bias)
            elif isinstance(module, (nn.Embedding, TritonEmbedding)):
                nn.init.normal_(module.weight, mean=0.0, std=std)

    @classmethod
    def from_reference_model(cls, reference_model: nn.Module, config: QwenTritonConfig) -> "QwenTritonForCausalLM":
        inst = cls.__new__(cls)
        nn.Module.__init__(inst)
        inst.config = config
        inst.backend = "ref"
        inst.ref_model = reference_model
        return inst

    @classmethod
    def from_config(cls, config, backend: str = "triton", init_weights: bool = True) -> "QwenTritonForCausalLM":
        cfg = config if isinstance(config, QwenTritonConfig) else QwenTritonConfig.from_hf_config(config)
        if backend != "triton":
            raise ValueError("from_config currently supports backend='triton' only")
        return cls(cfg, backend=backend, init_weights=init_weights)

    @classmethod
    def from_pretrained_hf(cls, model_id: str, backend: str = "triton", device="cpu", dtype=None):
        from qwen_triton.loaders import load_config_dict, load_hf_weights_into_model, ensure_local_model_path

        cfg = QwenTritonConfig.from_hf_config(load_config_dict(model_id))
        parsed = _parse_dtype(dtype) or torch.float32
        if backend == "ref":
            from transformers import AutoModelForCausalLM

            ref = AutoModelForCausalLM.from_pretrained(model_id, trust_remote_code=True, torch_dtype=parsed)
            return cls.from_reference_model(ref.to(device), cfg)
        path = ensure_local_model_path(model_id, include_weights=True)
        inst = cls.from_config(cfg, backend="triton", init_weights=False)
        inst.to(dtype=parsed)
        load_hf_weights_into_model(inst, path)
        inst.to(device=device)
        inst.eval()
        return inst

    def forward(self, input_ids=None, attention_mask=None, position_ids=None, past_key_values=None, inputs_embeds=None,
                labels=None, use_cache=None, cache_position=None, logits_to_keep: int | torch.Tensor = 0,
                output_router_logits: bool = False, **kwargs: Any) -> CausalLMOutputWithPast:
        if self.backend == "ref":
            return self.ref_model(input_ids=input_ids, attention_mask=attention_mask, position_ids=position_ids,
                                  past_key_values=past_key_values, inputs_embeds=inputs_embeds, labels=labels,
                                  use_cache=use_cache, cache_position=cache_position, **kwargs)
        outputs = self.model(input_ids=input_ids, attention_mask=attention_mask, position_ids=position_ids,
                             past_key_values=past_key_values, inputs_embeds=inputs_embeds, use_cache=use_cache,
                             cache_position=cache_position, output_router_logits=output_router_logits, **kwargs)
        hidden = outputs.last_hidden_state
        if isinstance(logits_to_keep, int) and logits_to_keep > 0:
            hidden = hidden[:, -logits_to_keep:, :]
        elif not isinstance(logits_to_keep, int):
            hidden = hidden[:, logits_to_keep, :]
        logits = self.lm_head(hidden)
        loss = _loss_fn(logits, labels) if labels is not None else None
        result = CausalLMOutputWithPast(loss=loss, logits=logits, past_key_values=outputs.past_key_values,
                                        hidden_states=None, attentions=None)
        if output_router_logits:
            result["router_logits"] = outputs.router_logits
        return result

    def new_cache(self, batch: int, capacity: int, dtype: torch.dtype, device) -> QwenTritonCache:
        """A cache with every attention layer preallocated to ``capacity`` positions."""
        cfg = self.config
        cache = QwenTritonCache(cfg.num_hidden_layers, cfg.layer_types, max_cache_len=cfg.max_position_embeddings)
        for i, kind in enumerate(cfg.layer_types):
            if kind != "linear_attention":
                cache.reserve(i, batch, cfg.num_key_value_heads, capacity, cfg.head_dim, dtype, device)
        return cache

    @torch.no_grad()
    def greedy_generate(self, input_ids: torch.LongTensor, attention_mask: torch.Tensor | None = None,
                        max_new_tokens: int = 16, use_graph: bool = False) -> torch.LongTensor:
        """Greedy decoding (reference: qwen_triton/models/core.py:378-410).

        ``use_graph=True`` (GPU, bf16/fp16, no padding mask) runs the prefill and every decode step
        as replays of two HIP graphs captured once per generation shape (``greedy_graphs``): the
        step reads its cache position and valid lengths from device memory, picks the next token
        and advances that state itself, so there is no host work between tokens. The eager loop
        of a model that qualifies for the graphs decodes through the same device state (a
        ``StaticDecode`` on its cache, advanced by two small device ops per token) without
        capturing it, so both run the same kernels with the same arguments and give the same
        tokens at every cache length.
        """
        if self.backend == "ref" and hasattr(self.ref_model, "generate"):
            return self.ref_model.generate(input_ids=input_ids, attention_mask=attention_mask,
                                           max_new_tokens=max_new_tokens, do_sample=False)
        # one device sync for the whole generation: an all-ones mask (and the ones appended to
        # it) means plain causal attention, so the steps run without it and without a check each
        trivial_mask = QwenTritonModel._mask_is_trivial(attention_mask)
        if use_graph and max_new_tokens > 2 and self._graph_decode_ok(input_ids, trivial_mask):
            return self._greedy_generate_graph(input_ids, max_new_tokens)
        generated = input_ids
        running_mask = None if trivial_mask else attention_mask
        cache = None
        if max_new_tokens > 0:
            dtype = self.lm_head.weight.dtype
            cache = self.new_cache(input_ids.shape[0], input_ids.shape[1] + max_new_tokens, dtype, input_ids.device)
        # decode steps through device-side state, as the captured step does (see the docstring)
        static = None
        if max_new_tokens > 1 and self._graph_decode_ok(input_ids, trivial_mask):
            batch, prompt = input_ids.shape
            static = StaticDecode(positions=torch.full((1,), prompt, dtype=torch.long, device=input_ids.device),
                                  seqlens=torch.full((batch,), prompt + 1, dtype=torch.int32, device=input_ids.device))
        for i in range(max_new_tokens):
            step_ids = generated if i == 0 else generated[:, -1:]
            if i > 0 and static is not None:
                cache.static = static
            try:
                out = self(input_ids=step_ids, attention_mask=running_mask, past_key_values=cache, use_cache=True,
                           logits_to_keep=1)
            finally:
                cache.static = None
            if i > 0 and static is not None:
                static.positions.add_(1)
                static.seqlens.add_(1)
            next_token = out.logits[:, -1].argmax(dim=-1, keepdim=True)
            generated = torch.cat((generated, next_token), dim=-1)
            if running_mask is not None:
                running_mask = torch.cat((running_mask, torch.ones_like(next_token, dtype=running_mask.dtype)), dim=-1)
        return generated

    def _graph_decode_ok(self, input_ids: torch.Tensor, trivial_mask: bool) -> bool:
        from qwen_triton import _native

        cfg = self.config
        dtype = self.lm_head.weight.dtype
        return (input_ids.is_cuda and dtype in (torch.bfloat16, torch.float16) and _native.available()
                and not cfg.attn_output_gate and all(t == "full_attention" for t in cfg.layer_types)
                and trivial_mask)

    def greedy_graphs(self, batch: int, prompt: int, max_new_tokens: int):
        """The captured-graph runner (``models.graphs.GreedyGraphs``) for this generation shape,
        created on first use and kept (the four most recent shapes; ``release_graphs`` frees them).
        Runners are keyed on the parameters' storage and version counters too, so parameters that
        are replaced or updated in place (a checkpoint ``copy_``, an optimizer step) get new graphs,
        captured over freshly derived tensors (norm-folded weights); a runner keeps the derived
        tensors its graphs read alive itself."""
        from collections import OrderedDict

        from qwen_triton.models.graphs import GreedyGraphs

        w = self.lm_head.weight
        key = (batch, prompt, max_new_tokens, w.dtype, w.device, _matmul.FOLD_NORM_WEIGHTS,
               tuple((p.data_ptr(), p._version) for p in self.parameters()))
        runners = self.__dict__.setdefault("_graph_runners", OrderedDict())
        runner = runners.get(key)
        if runner is None:
            while len(runners) >= 4:
                runners.popitem(last=False)
            runner = runners[key] = GreedyGraphs(self, batch, prompt, max_new_tokens, w.dtype, w.device)
        runners.move_to_end(key)
        return runner

    def release_graphs(self) -> None:
        """Drop the captured generation graphs and their caches."""
        self.__dict__.pop("_graph_runners", None)

    def release_folded_weights(self) -> int:
        """Free the norm-folded copies of the q/k/v and gate/up weights that batched inference
        keeps (about 0.59 GB at Qwen3-0.6B; ``kernels.matmul.FOLD_NORM_WEIGHTS`` turns them off),
        and the captured graphs that read them. Returns the bytes released."""
        self.release_graphs()
        return _matmul.release_folded_weights(self)

    @torch.no_grad()
    def _greedy_generate_graph(self, input_ids: torch.LongTensor, max_new_tokens: int) -> torch.LongTensor:
        return self.greedy_graphs(input_ids.shape[0], input_ids.shape[1], max_new_tokens).generate(input_ids)
