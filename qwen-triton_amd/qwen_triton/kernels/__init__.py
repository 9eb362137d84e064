"""Operator API of the MI355X stack (same names and signatures as the reference's
qwen_triton/kernels/__init__.py:1-32); every op runs on libqwen_hip.so for GPU
tensors."""
from .cache import append_attention_kv, write_attention_kv
from .cross_entropy import triton_cross_entropy
from .embedding import triton_embedding
from .flash_attention import triton_flash_attention
from .linear_attention import gated_delta_rule_sequence
from .linear_cross_entropy import fused_linear_cross_entropy
from .matmul import triton_matmul
from .moe_routing import triton_index_add, triton_one_hot, triton_topk
from .residual_add import residual_add
from .rmsnorm import rmsnorm
from .rope import apply_rope
from .sigmoid_mul import sigmoid_mul
from .softmax import triton_softmax
from .swiglu import silu_mul

__all__ = [
    "append_attention_kv",
    "write_attention_kv",
    "triton_cross_entropy",
    "triton_embedding",
    "triton_flash_attention",
    "gated_delta_rule_sequence",
    "fused_linear_cross_entropy",
    "triton_matmul",
    "triton_index_add",
    "triton_one_hot",
    "triton_topk",
    "residual_add",
    "rmsnorm",
    "apply_rope",
    "sigmoid_mul",
    "triton_softmax",
    "silu_mul",
]
