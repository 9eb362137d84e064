"""Shared helpers for the parity tests."""
from __future__ import annotations

import torch

BF16_TOL = dict(atol=2e-2, rtol=2e-2)   # reference bf16 band (tests/test_kernels.py:150-163)
F32_TOL = dict(atol=1e-4, rtol=1e-4)    # reference fp32 band (tests/test_kernels.py:23-28)


def close(actual: torch.Tensor, expected: torch.Tensor, **tol) -> None:
    torch.testing.assert_close(actual.detach().cpu().to(torch.float64), expected.detach().cpu().to(torch.float64),
                               **tol)


def tol_for(dtype: torch.dtype) -> dict:
    return F32_TOL if dtype == torch.float32 else BF16_TOL


def native_calls(name: str) -> int:
    from qwen_triton import _native

    return _native.CALLS[name]
