from .config import QwenTritonConfig

__all__ = ["QwenTritonConfig"]
