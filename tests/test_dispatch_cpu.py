"""Host-side dispatch rules, exercised on the CPU with stand-in kernels.

* RoPE backend routing (the reference's backend ladder, qwen_triton/kernels/rope.py:123-300):
  one test per strict / fallback branch, with the GPU routes replaced by recording fakes that
  compute the exact result, so the branch taken is observable without a GPU.
* Capability gaps versus kernel failures (qwen_triton/kernels/_common.py): inputs outside what
  the HIP kernels serve run on torch for that call only; a kernel failure disables the kernel.
"""
from __future__ import annotations

import warnings

import pytest
import torch

from oracle import ops as O
from qwen_triton import _native
from qwen_triton import kernels as K
from qwen_triton.kernels import _common
from qwen_triton.kernels import rope as R


class _Fakes:
    def __init__(self):
        self.hip = 0
        self.op = 0
        self.op_loads = True
        self.hip_error: Exception | None = None
        self.op_error: Exception | None = None


@pytest.fixture
def gpu_routes(monkeypatch):
    """Make CPU tensors look like GPU tensors to the router; the routes record their calls."""
    f = _Fakes()
    monkeypatch.delenv("QWEN_TRITON_STRICT", raising=False)
    monkeypatch.delenv("QWEN_TRITON_ROPE_BACKEND", raising=False)
    monkeypatch.setattr(R, "_on_gpu", lambda *t: True)
    monkeypatch.setattr(_native, "available", lambda: True)
    R._GUARD.reset()
    R._HANDOVER_WARNED.clear()

    def hip(x, cos, sin, neg_sin=False):
        f.hip += 1
        if f.hip_error is not None:
            raise f.hip_error
        return O.rope(x, cos, -sin if neg_sin else sin)

    def op_pair(q, k, cos, sin):
        f.op += 1
        if f.op_error is not None:
            raise f.op_error
        return O.rope(q, cos, sin), O.rope(k, cos, sin)

    def op_single(x, cos, sin):
        f.op += 1
        if f.op_error is not None:
            raise f.op_error
        return O.rope(x, cos, sin)

    monkeypatch.setattr(R, "rope_tensor", hip)
    monkeypatch.setattr(R, "apply_rope_cuda_op", op_pair)
    monkeypatch.setattr(R, "_custom_op_single", op_single)
    monkeypatch.setattr(R, "load_rope_cuda_op", lambda verbose=False: f.op_loads)
    yield f
    R._GUARD.reset()
    R._HANDOVER_WARNED.clear()


def _inputs(grad=False):
    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, 4, 5, 16, generator=g, dtype=torch.float64).requires_grad_(grad)
    k = torch.randn(2, 2, 5, 16, generator=g, dtype=torch.float64).requires_grad_(grad)
    cos = torch.randn(2, 5, 8, generator=g, dtype=torch.float64)
    sin = torch.randn(2, 5, 8, generator=g, dtype=torch.float64)
    return q, k, cos, sin


def _check_forward(out, q, k, cos, sin):
    torch.testing.assert_close(out[0], O.rope(q.detach(), cos, sin))
    torch.testing.assert_close(out[1], O.rope(k.detach(), cos, sin))


def _fallback_warnings(rec):
    return [w for w in rec if "[Qwen-Triton fallback]" in str(w.message)]


def test_rope_backend_resolution(monkeypatch):
    from qwen_triton.kernels.rope import _resolve_backend

    monkeypatch.delenv("QWEN_TRITON_ROPE_BACKEND", raising=False)
    assert _resolve_backend(None, None) == "triton"
    assert _resolve_backend(False, None) == "torch"
    assert _resolve_backend(False, "AUTO") == "auto"  # an explicit backend wins over use_triton
    monkeypatch.setenv("QWEN_TRITON_ROPE_BACKEND", "CUDA_OP")
    assert _resolve_backend(None, None) == "cuda_op"
    with pytest.raises(ValueError, match="Unsupported RoPE backend"):
        K.apply_rope(*_inputs(), backend="bogus")


def test_rope_triton_runs_the_hip_route(gpu_routes):
    q, k, cos, sin = _inputs()
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        out = K.apply_rope(q, k, cos, sin)
    _check_forward(out, q, k, cos, sin)
    assert gpu_routes.hip == 2 and gpu_routes.op == 0
    assert not _fallback_warnings(rec)


def test_rope_hip_failure_is_sticky_and_warns_once(gpu_routes):
    q, k, cos, sin = _inputs()
    gpu_routes.hip_error = RuntimeError("launch failed")
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        out = K.apply_rope(q, k, cos, sin)
        out2 = K.apply_rope(q, k, cos, sin)
    _check_forward(out, q, k, cos, sin)
    _check_forward(out2, q, k, cos, sin)
    assert gpu_routes.hip == 1  # the second call no longer tries the kernel
    assert not R._GUARD.runtime_ok
    msgs = [str(w.message) for w in _fallback_warnings(rec)]
    assert sum("HIP kernel unavailable" in m for m in msgs) == 1


def test_rope_hip_failure_raises_in_strict_mode(gpu_routes, monkeypatch):
    monkeypatch.setenv("QWEN_TRITON_STRICT", "1")
    gpu_routes.hip_error = RuntimeError("launch failed")
    with pytest.raises(RuntimeError, match="strict"):
        K.apply_rope(*_inputs())


def test_rope_unsupported_inputs_do_not_disable_the_kernel(gpu_routes):
    q, k, cos, sin = _inputs()
    gpu_routes.hip_error = _native.Unsupported("rope cos/sin batch 3 must be 1 or 2")
    with warnings.catch_warnings(record=True):
        warnings.simplefilter("always")
        out = K.apply_rope(q, k, cos, sin)
    _check_forward(out, q, k, cos, sin)
    assert R._GUARD.runtime_ok
    gpu_routes.hip_error = None
    K.apply_rope(q, k, cos, sin)
    assert gpu_routes.hip == 3  # one failed attempt, then both tensors of the next call


def test_rope_cuda_op_route_and_its_backward(gpu_routes):
    q, k, cos, sin = _inputs(grad=True)
    out = K.apply_rope(q, k, cos, sin, backend="cuda_op")
    _check_forward(out, q, k, cos, sin)
    assert gpu_routes.op == 1 and gpu_routes.hip == 0
    gq, gk = torch.randn_like(out[0]), torch.randn_like(out[1])
    torch.autograd.backward(out, (gq, gk))
    torch.testing.assert_close(q.grad, O.rope_backward(gq, cos, sin))
    torch.testing.assert_close(k.grad, O.rope_backward(gk, cos, sin))
    assert gpu_routes.op == 3 and gpu_routes.hip == 0  # the backward retraces the custom op route


def test_rope_cuda_op_unloadable_hands_over_to_hip(gpu_routes):
    gpu_routes.op_loads = False
    q, k, cos, sin = _inputs()
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        out = K.apply_rope(q, k, cos, sin, backend="cuda_op")
    _check_forward(out, q, k, cos, sin)
    assert gpu_routes.hip == 2
    assert any("custom op unavailable" in str(w.message) for w in _fallback_warnings(rec))


def test_rope_cuda_op_unloadable_raises_in_strict_mode(gpu_routes, monkeypatch):
    monkeypatch.setenv("QWEN_TRITON_STRICT", "1")
    gpu_routes.op_loads = False
    with pytest.raises(RuntimeError, match="custom_op route unavailable"):
        K.apply_rope(*_inputs(), backend="cuda_op")


def test_rope_auto_skips_an_unloadable_op_even_in_strict_mode(gpu_routes, monkeypatch):
    monkeypatch.setenv("QWEN_TRITON_STRICT", "1")
    gpu_routes.op_loads = False
    q, k, cos, sin = _inputs()
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        out = K.apply_rope(q, k, cos, sin, backend="auto")
    _check_forward(out, q, k, cos, sin)
    assert gpu_routes.hip == 2 and not _fallback_warnings(rec)


def test_rope_custom_op_failure(gpu_routes, monkeypatch):
    gpu_routes.op_error = RuntimeError("op failed")
    q, k, cos, sin = _inputs()
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        out = K.apply_rope(q, k, cos, sin, backend="auto")
    _check_forward(out, q, k, cos, sin)
    assert gpu_routes.hip == 2
    assert any("custom op failed" in str(w.message) for w in _fallback_warnings(rec))
    # "auto" does not require the op, "cuda_op" does
    monkeypatch.setenv("QWEN_TRITON_STRICT", "1")
    K.apply_rope(q, k, cos, sin, backend="auto")
    with pytest.raises(RuntimeError, match="custom op failed"):
        K.apply_rope(q, k, cos, sin, backend="cuda_op")


def test_rope_backward_hip_failure_falls_back_to_torch(gpu_routes):
    q, k, cos, sin = _inputs(grad=True)
    out = K.apply_rope(q, k, cos, sin)
    gpu_routes.hip_error = RuntimeError("backward launch failed")
    gq, gk = torch.randn_like(out[0]), torch.randn_like(out[1])
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        torch.autograd.backward(out, (gq, gk))
    torch.testing.assert_close(q.grad, O.rope_backward(gq, cos, sin))
    torch.testing.assert_close(k.grad, O.rope_backward(gk, cos, sin))
    assert not R._GUARD.runtime_ok
    assert _fallback_warnings(rec)


def test_rope_cpu_tensors(monkeypatch):
    """Off the GPU: torch without warnings, except that strict mode refuses the accelerated backends
    (as the reference does for CPU tensors)."""
    monkeypatch.delenv("QWEN_TRITON_STRICT", raising=False)
    R._HANDOVER_WARNED.clear()
    q, k, cos, sin = _inputs()
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        for backend in ("triton", "auto", "cuda_op", "torch"):
            _check_forward(K.apply_rope(q, k, cos, sin, backend=backend), q, k, cos, sin)
    assert not _fallback_warnings(rec)
    monkeypatch.setenv("QWEN_TRITON_STRICT", "1")
    _check_forward(K.apply_rope(q, k, cos, sin, backend="torch"), q, k, cos, sin)
    for backend in ("triton", "auto", "cuda_op"):
        with pytest.raises(RuntimeError, match="strict"):
            K.apply_rope(q, k, cos, sin, backend=backend)


# ---------------------------------------------------------------------------
# capability gaps are not kernel failures
# ---------------------------------------------------------------------------
def test_guard_unsupported_is_not_sticky(monkeypatch):
    monkeypatch.delenv("QWEN_TRITON_STRICT", raising=False)
    guard = _common.OpGuard("Probe")
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        guard.failed(_native.Unsupported("fp32 inputs"))
        guard.failed(_native.Unsupported("fp32 inputs"))
    assert guard.runtime_ok
    assert len(_fallback_warnings(rec)) == 1  # once per distinct reason
    monkeypatch.setenv("QWEN_TRITON_STRICT", "1")
    with pytest.raises(RuntimeError, match="not served"):
        guard.failed(_native.Unsupported("fp32 inputs"))
    assert guard.runtime_ok
    monkeypatch.delenv("QWEN_TRITON_STRICT")
    with warnings.catch_warnings(record=True):
        warnings.simplefilter("always")
        guard.failed(RuntimeError("launch failed"))
    assert not guard.runtime_ok


def test_library_argument_rejections_are_unsupported():
    # QH_E_ARG / QH_E_DTYPE come from checks that run before any launch
    if not _native.available():
        pytest.skip("library not built")
    with pytest.raises(_native.Unsupported):
        _native.call("qh_add", None, None, None, -1, _native.BF16, None)
    with pytest.raises(_native.Unsupported):
        _native.dtype_code(torch.int32)


def test_flash_attention_on_cpu_tensors_forced_native_keeps_the_kernel_enabled(monkeypatch):
    """use_triton=True with tensors the kernels cannot take runs torch for that call and leaves the
    operator on the kernels (the reference's flag is sticky only on a real kernel failure)."""
    if not _native.available():
        pytest.skip("library not built")
    from qwen_triton.kernels import flash_attention as FA

    monkeypatch.delenv("QWEN_TRITON_STRICT", raising=False)
    FA._GUARD.reset()
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 4, 6, 16, generator=g)
    k = torch.randn(1, 2, 6, 16, generator=g)
    v = torch.randn(1, 2, 6, 16, generator=g)
    with warnings.catch_warnings(record=True):
        warnings.simplefilter("always")
        out = K.triton_flash_attention(q, k, v, 0.25, True, 2, use_triton=True)
    torch.testing.assert_close(out, O.attention(q, k, v, 0.25, True, 2)[0].float(), rtol=1e-5, atol=1e-5)
    assert FA._GUARD.runtime_ok
    FA._GUARD.reset()


def test_flash_backward_fallback_keeps_the_bottom_right_mask():
    from qwen_triton.kernels.flash_attention import _torch_attention_offset

    g = torch.Generator().manual_seed(2)
    q = torch.randn(1, 4, 3, 8, generator=g, dtype=torch.float64)
    k = torch.randn(1, 2, 7, 8, generator=g, dtype=torch.float64)
    v = torch.randn(1, 2, 7, 8, generator=g, dtype=torch.float64)
    out = _torch_attention_offset(q, k, v, 0.3, True, 2, 4)
    ref = O.attention(q, k, v, 0.3, True, 2, causal_offset=4)[0]
    torch.testing.assert_close(out, ref.to(out.dtype))


def test_pack_key_bits_layout_cpu():
    """Bit j % 64 of word j // 64 is key j (bit 63 is the sign bit); keys past Sk are clear."""
    from qwen_triton.kernels.flash_attention import pack_key_bits

    kv = torch.zeros(2, 130, dtype=torch.int64)
    kv[0, [0, 63, 64, 129]] = 1
    kv[1] = 1
    assert pack_key_bits(kv).tolist() == [[1 - (1 << 63), 1, 2], [-1, -1, 3]]


def test_structured_mask_matches_the_additive_mask_and_keeps_the_step_start():
    """The structured mask's dense form is the additive mask for the step's first cache length, even
    when a layer has appended its keys before asking for it; its key rows prepend ones for cached
    keys the 2-D mask does not cover; the kernel arguments are refused for other shapes."""
    from types import SimpleNamespace

    from qwen_triton.models.core import _build_causal_mask, _structured_mask

    cache = SimpleNamespace(n=5)
    cache.get_seq_length = lambda: cache.n
    am = torch.tensor([[0, 0, 1, 1, 1], [1, 1, 1, 1, 1]])  # covers 5 of the 8 keys (3 cached)
    pos = torch.arange(5, 8)
    mask = _structured_mask(am, 2, pos, torch.device("cpu"), cache, 4, True)
    expect = _build_causal_mask(am, 2, pos, torch.device("cpu"), 5, 4)
    cache.n = 8  # the first layer wrote the step's keys
    assert torch.equal(mask.dense(), expect)
    assert mask.key_valid.tolist() == [[1, 1, 1, 0, 0, 1, 1, 1], [1] * 8]
    q, k = torch.zeros(2, 4, 3, 8), torch.zeros(2, 2, 8, 8)
    bits, window, offset = mask.kernel_args(q, k)
    assert bits.tolist() == [[0b11100111], [0b11111111]] and window == 4 and offset == 5
    assert mask.kernel_args(q, torch.zeros(2, 2, 9, 8)) is None  # keys beyond the step's length
    blocked = _structured_mask(am, 2, pos, torch.device("cpu"), cache, None, False)
    assert blocked.kernel_args(q, torch.zeros(2, 2, 11, 8)) is None  # caller-given positions
    # the dense form: query 0 (position 5) sees keys 2..5 by the window, minus the padding of row 0
    visible = expect[0, 0, 0] == 0
    assert visible.tolist() == [False, False, True, False, False, True, False, False]
