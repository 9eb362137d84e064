"""The C-ABI library and the Python dispatch layer (CPU only: no kernel is launched here)."""
from __future__ import annotations

import ctypes
import re
import warnings
from pathlib import Path

import pytest
import torch

from qwen_triton import _native
from qwen_triton import kernels as K
from qwen_triton.kernels import _common

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = "\n".join(p.read_text() for p in (ROOT / "include").glob("*.h"))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(qh_\w+)\s*\(", text)


def test_library_loads_and_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    names = _declared()
    assert len(names) >= 30
    for name in names:
        assert hasattr(lib, name), name
    assert _native.available()
    assert "gfx950" in _native.version()


def test_header_signatures_bind():
    sigs = _native.parse_header()
    assert sigs["qh_gemm"] == ("i", "iilllplplplpiip")
    assert sigs["qh_last_error"] == ("s", "")
    assert set(sigs) == set(_declared())


def test_workspace_queries_are_host_only():
    assert _native.call("qh_rmsnorm_bwd_workspace", 16384, 1024, _native.BF16) > 0
    # id sort space: keys and token positions, in and out (no per-row table)
    assert _native.call("qh_embedding_bwd_workspace", 16384, 151936) >= 4 * 16384 * 4
    # Delta and log2-scale LSE per query, rows padded to a multiple of 64 plus one 64-query tile
    assert _native.call("qh_flash_bwd_workspace", 8, 16, 4096) == 2 * 8 * 16 * (4096 + 64) * 4
    assert _native.call("qh_flash_bwd_workspace", 1, 2, 65) == 2 * 1 * 2 * (128 + 64) * 4
    # 64 sequences x 8 kv-heads at head dim 128: one workgroup per pair, partials combined on chip
    assert _native.call("qh_flash_decode_workspace", 64, 16, 8, 2049, 128) == 0
    assert _native.call("qh_flash_decode_workspace", 8, 32, 8, 2900, 128) > 0


def test_argument_errors_are_reported_without_launching():
    with pytest.raises(_native.NativeError, match="rotary dim"):
        _native.call("qh_rope", 0, 1, 1, 1, 1, 0, 0, 1, 1, 1, 1, 0, 1, 1, 1, 4, 3, 0, _native.BF16, _native.BF16, 0)
    with pytest.raises(_native.NativeError, match="k=5 > C=4"):
        _native.call("qh_topk", 0, 0, 0, 1, 4, 5, _native.F32, 0)
    with pytest.raises(_native.NativeError, match="N and ldc multiples of 8"):  # 16-byte output rows
        _native.call("qh_moe_down", 0, 8, 1, 8, 0, 8, 100, 0, 0, 1, 0, 100, 0, _native.BF16, 0)
    with pytest.raises(_native.NativeError, match="head dim"):
        _native.call("qh_flash_fwd", 0, 0, 0, 8, 0, 0, 0, 8, 0, 0, 0, 8, 0, 0, 0, 8, 0, 1, 1, 1, 1, 1, 200, 1.0, 1,
                     0, _native.BF16, 0)


def test_cpu_tensors_use_torch_path_like_the_reference():
    x, w = torch.randn(3, 8), torch.randn(8)
    torch.testing.assert_close(K.rmsnorm(x, w), K.rmsnorm(x, w, use_triton=False))


def test_forced_native_on_cpu_falls_back_with_one_warning(monkeypatch):
    monkeypatch.delenv("QWEN_TRITON_STRICT", raising=False)
    from qwen_triton.kernels import swiglu

    swiglu._GUARD.reset()
    try:
        with warnings.catch_warnings(record=True) as rec:
            warnings.simplefilter("always")
            a, b = torch.randn(4), torch.randn(4)
            out = K.silu_mul(a, b, use_triton=True)
            out2 = K.silu_mul(a, b, use_triton=True)
        torch.testing.assert_close(out, torch.nn.functional.silu(a) * b)
        torch.testing.assert_close(out2, out)
        msgs = [str(r.message) for r in rec if "[Qwen-Triton fallback]" in str(r.message)]
        assert len(msgs) == 1
        # CPU tensors are inputs the kernels do not take, not a kernel failure: the operator stays on
        # the kernels for later GPU calls (the reference's flag would stick here)
        assert swiglu._GUARD.runtime_ok is True
    finally:
        swiglu._GUARD.reset()


def test_strict_mode_raises(monkeypatch):
    monkeypatch.setenv("QWEN_TRITON_STRICT", "1")
    from qwen_triton.kernels import softmax

    softmax._GUARD.reset()
    try:
        with pytest.raises(RuntimeError, match="strict"):
            K.triton_softmax(torch.randn(2, 3), use_triton=True)
    finally:
        softmax._GUARD.reset()


def test_missing_library_is_loud_for_gpu_tensors(monkeypatch):
    guard = _common.OpGuard("Probe")

    class FakeCuda:
        is_cuda = True

    monkeypatch.setattr(_native, "available", lambda: False)
    with pytest.raises(RuntimeError, match="could not be loaded"):
        guard.use_native(None, FakeCuda())
