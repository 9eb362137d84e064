from .core import QwenTritonForCausalLM

__all__ = ["QwenTritonForCausalLM"]
