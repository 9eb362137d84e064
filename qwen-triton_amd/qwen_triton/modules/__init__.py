from .attention import QwenFullAttention, repeat_kv
from .cache import QwenTritonCache
from .embedding import TritonEmbedding
from .linear import TritonLinear
from .linear_attention import Qwen3NextLinearAttention
from .mlp import QwenMLP
from .moe import QwenSparseMoeBlock
from .norms import QwenRMSNorm, QwenRMSNormGated
from .rotary import QwenRotaryEmbedding, apply_rotary_pos_emb

__all__ = [
    "QwenFullAttention",
    "QwenTritonCache",
    "Qwen3NextLinearAttention",
    "QwenMLP",
    "QwenSparseMoeBlock",
    "QwenRMSNorm",
    "QwenRMSNormGated",
    "QwenRotaryEmbedding",
    "TritonEmbedding",
    "TritonLinear",
    "apply_rotary_pos_emb",
    "repeat_kv",
]
