"""Normalised model configuration for the Qwen3 family.

Reference: qwen_triton/configs/config.py:1-203 (layer-type defaults :5-26, family
detection :29-41, dataclass :44-110, ``from_hf_config`` :111-200). Accepts an HF
config object (anything with ``to_dict``) or a plain mapping, with or without a
nested ``text_config``; rope parameters may sit at top level or in
``rope_parameters`` (transformers >= 5).
"""
from __future__ import annotations

from dataclasses import asdict, dataclass, field
from typing import Any, Mapping

_NEXT_TYPES = {"qwen3_next", "qwen3_5_text", "qwen3_5_moe_text"}
_QWEN35_TYPES = {"qwen3_next", "qwen3_5", "qwen3_5_text", "qwen3_5_moe", "qwen3_5_moe_text"}


def _family(model_type: str, cfg: Mapping[str, Any]) -> str:
    if model_type == "qwen3":
        return "qwen3_dense"
    if model_type == "qwen3_moe":
        return "qwen3_moe"
    if model_type in _QWEN35_TYPES:
        experts = int(cfg.get("num_experts") or cfg.get("num_local_experts") or 0)
        shared = int(cfg.get("shared_expert_intermediate_size") or 0)
        moe = experts > 0 or shared > 0 or "moe" in model_type
        return "qwen35_text_moe" if moe else "qwen35_text_dense"
    raise ValueError(f"Unsupported Qwen model_type: {model_type}")


def _layer_types(model_type: str, n_layers: int, cfg: Mapping[str, Any]) -> list[str]:
    if model_type in _NEXT_TYPES:
        interval = int(cfg.get("full_attention_interval") or 4)
        return ["full_attention" if (i + 1) % interval == 0 else "linear_attention" for i in range(n_layers)]
    window = cfg.get("sliding_window")
    if cfg.get("use_sliding_window") and window is not None:
        cutoff = cfg.get("max_window_layers")
        cutoff = n_layers if cutoff is None else int(cutoff)
        return ["sliding_attention" if i >= cutoff else "full_attention" for i in range(n_layers)]
    return ["full_attention"] * n_layers


@dataclass
class QwenTritonConfig:
    family: str
    source_model_type: str
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    hidden_act: str = "silu"
    max_position_embeddings: int = 32768
    initializer_range: float = 0.02
    rms_norm_eps: float = 1e-6
    use_cache: bool = True
    tie_word_embeddings: bool = False
    rope_theta: float = 10000.0
    attention_bias: bool = False
    attention_dropout: float = 0.0
    pad_token_id: int | None = None
    bos_token_id: int | None = None
    eos_token_id: int | None = None
    torch_dtype: str | None = None
    use_sliding_window: bool = False
    sliding_window: int | None = None
    max_window_layers: int | None = None
    layer_types: list[str] = field(default_factory=list)
    partial_rotary_factor: float = 1.0
    attn_output_gate: bool = False
    norm_one_plus: bool = False
    linear_conv_kernel_dim: int = 4
    linear_key_head_dim: int = 128
    linear_value_head_dim: int = 128
    linear_num_key_heads: int = 0
    linear_num_value_heads: int = 0
    decoder_sparse_step: int = 1
    moe_intermediate_size: int = 0
    shared_expert_intermediate_size: int = 0
    num_experts_per_tok: int = 0
    num_experts: int = 0
    norm_topk_prob: bool = False
    router_aux_loss_coef: float = 0.0
    mlp_only_layers: list[int] = field(default_factory=list)
    raw_config: dict[str, Any] = field(default_factory=dict, repr=False)

    @property
    def is_moe(self) -> bool:
        return self.family in {"qwen3_moe", "qwen35_text_moe"}

    @property
    def is_qwen35_family(self) -> bool:
        return self.family in {"qwen35_text_dense", "qwen35_text_moe"}

    @property
    def rotary_dim(self) -> int:
        dim = max(2, int(self.head_dim * self.partial_rotary_factor))
        return dim - (dim % 2)

    @classmethod
    def from_hf_config(cls, hf_config: Any) -> "QwenTritonConfig":
        if hasattr(hf_config, "to_dict"):
            raw = dict(hf_config.to_dict())
        elif isinstance(hf_config, Mapping):
            raw = dict(hf_config)
        else:
            raise TypeError(f"Unsupported config type: {type(hf_config)!r}")
        cfg = dict(raw.get("text_config") or raw)
        model_type = str(cfg.get("model_type") or raw.get("model_type"))
        family = _family(model_type, cfg)
        rope = dict(cfg.get("rope_parameters") or {})
        n_layers = int(cfg["num_hidden_layers"])
        heads = int(cfg["num_attention_heads"])
        head_dim = int(cfg.get("head_dim") or int(cfg["hidden_size"]) // heads)
        gate = cfg.get("attn_output_gate")
        if gate is None:
            gate = model_type in _NEXT_TYPES
        window = cfg.get("sliding_window")
        max_window = cfg.get("max_window_layers")

        def pick(name: str, default: Any) -> Any:
            return cfg.get(name, raw.get(name, default))

        config = cls(
            family=family,
            source_model_type=model_type,
            vocab_size=int(cfg["vocab_size"]),
            hidden_size=int(cfg["hidden_size"]),
            intermediate_size=int(cfg.get("intermediate_size") or 0),
            num_hidden_layers=n_layers,
            num_attention_heads=heads,
            num_key_value_heads=int(cfg.get("num_key_value_heads") or heads),
            head_dim=head_dim,
            hidden_act=str(cfg.get("hidden_act", "silu")),
            max_position_embeddings=int(cfg.get("max_position_embeddings", 32768)),
            initializer_range=float(cfg.get("initializer_range", 0.02)),
            rms_norm_eps=float(cfg.get("rms_norm_eps", 1e-6)),
            use_cache=bool(cfg.get("use_cache", True)),
            tie_word_embeddings=bool(raw.get("tie_word_embeddings", cfg.get("tie_word_embeddings", False))),
            rope_theta=float(cfg.get("rope_theta") or rope.get("rope_theta") or 10000.0),
            attention_bias=bool(cfg.get("attention_bias", False)),
            attention_dropout=float(cfg.get("attention_dropout", 0.0)),
            pad_token_id=pick("pad_token_id", None),
            bos_token_id=pick("bos_token_id", None),
            eos_token_id=pick("eos_token_id", None),
            torch_dtype=str(cfg.get("torch_dtype") or cfg.get("dtype") or raw.get("torch_dtype") or ""),
            use_sliding_window=bool(cfg.get("use_sliding_window", False)),
            sliding_window=None if window is None else int(window),
            max_window_layers=None if max_window is None else int(max_window),
            layer_types=list(cfg.get("layer_types") or _layer_types(model_type, n_layers, cfg)),
            partial_rotary_factor=float(cfg.get("partial_rotary_factor") or rope.get("partial_rotary_factor") or 1.0),
            attn_output_gate=bool(gate),
            norm_one_plus=model_type in _NEXT_TYPES,
            linear_conv_kernel_dim=int(cfg.get("linear_conv_kernel_dim", 4)),
            linear_key_head_dim=int(cfg.get("linear_key_head_dim", head_dim)),
            linear_value_head_dim=int(cfg.get("linear_value_head_dim", head_dim)),
            linear_num_key_heads=int(cfg.get("linear_num_key_heads") or 0),
            linear_num_value_heads=int(cfg.get("linear_num_value_heads") or 0),
            decoder_sparse_step=int(cfg.get("decoder_sparse_step", 1)),
            moe_intermediate_size=int(cfg.get("moe_intermediate_size") or 0),
            shared_expert_intermediate_size=int(cfg.get("shared_expert_intermediate_size") or 0),
            num_experts_per_tok=int(cfg.get("num_experts_per_tok") or 0),
            num_experts=int(cfg.get("num_experts") or cfg.get("num_local_experts") or 0),
            norm_topk_prob=bool(cfg.get("norm_topk_prob", False)),
            router_aux_loss_coef=float(cfg.get("router_aux_loss_coef", 0.0)),
            mlp_only_layers=list(cfg.get("mlp_only_layers") or []),
            raw_config=raw,
        )
        if family == "qwen35_text_dense":
            config.num_experts = config.num_experts_per_tok = config.shared_expert_intermediate_size = 0
        return config

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)
