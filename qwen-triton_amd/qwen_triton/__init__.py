"""MI355X (gfx950) implementation of the Qwen-Triton operator stack.

Same import paths as the reference package: ``qwen_triton.kernels``,
``.modules``, ``.models``, ``.configs``, ``.ops``, ``.loaders``. GPU tensors run
on the hand-written HIP kernels of ``_lib/libqwen_hip.so``.
"""
from . import _native
from .configs import QwenTritonConfig
from .models import QwenTritonForCausalLM

__all__ = ["QwenTritonConfig", "QwenTritonForCausalLM", "_native"]
