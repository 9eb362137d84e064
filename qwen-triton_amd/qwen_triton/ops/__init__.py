from .rope_cuda import apply_rope_cuda_op, get_rope_cuda_op_error, load_rope_cuda_op

__all__ = ["apply_rope_cuda_op", "get_rope_cuda_op_error", "load_rope_cuda_op"]
