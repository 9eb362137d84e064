"""Dispatch policy shared by every operator wrapper.

Mirrors the reference's per-module convention (e.g.
qwen_triton/kernels/matmul.py:19-32, :235-255):

* ``use_triton=None`` selects the native kernel for device tensors, ``False``
  forces the torch path, ``True`` forces the native kernel;
* a kernel failure flips a sticky per-operator flag, then either raises
  ``RuntimeError`` (``QWEN_TRITON_STRICT=1``) or warns once with a
  ``[Qwen-Triton fallback]`` ``RuntimeWarning`` and uses torch from then on.

Inputs outside what the HIP kernels take (``Unsupported``: a dtype, head
dimension or layout the kernels do not serve, rejected before any launch) are
not kernel failures: that one call runs on torch (after a warning, or a
``RuntimeError`` in strict mode) and the flag stays set, so later calls with
supported inputs still reach the kernels.

One deliberate difference: if the native library itself cannot be loaded while
the inputs live on the GPU, the call raises instead of silently running torch,
so a GPU run can never pass on a fallback without anyone noticing.
"""
from __future__ import annotations

import os
import warnings

import torch

from .. import _native
from .._native import Unsupported  # noqa: F401  (re-exported for the wrappers)


def strict_mode() -> bool:
    return os.environ.get("QWEN_TRITON_STRICT") == "1"


class OpGuard:
    """Sticky runtime flag + warn-once state of one operator family."""

    def __init__(self, label: str) -> None:
        self.label = label
        self.runtime_ok = True
        self.warned = False
        self.unsupported_seen: set[str] = set()

    def use_native(self, use_triton: bool | None, *tensors: torch.Tensor | None) -> bool:
        if use_triton is None:
            use = all(t.is_cuda for t in tensors if t is not None)
        else:
            use = bool(use_triton)
        if not use or not self.runtime_ok:
            return False
        if not _native.available():
            raise RuntimeError(
                f"{self.label}: the HIP operator library is required for GPU tensors but could not be "
                f"loaded: {_native.load_error()!r}"
            )
        return True

    def failed(self, exc: BaseException, what: str = "kernel") -> None:
        """Record a failure; raises in strict mode, otherwise warns once.

        ``Unsupported`` inputs only route the current call to torch: the flag is left alone."""
        if isinstance(exc, Unsupported):
            if strict_mode():
                raise RuntimeError(f"{self.label}: inputs not served by the HIP {what} ({exc}) and strict "
                                   "mode is enabled.") from exc
            reason = str(exc)
            if reason not in self.unsupported_seen:
                self.unsupported_seen.add(reason)
                warnings.warn(f"[Qwen-Triton fallback] {self.label}: {reason}. This call uses torch.",
                              RuntimeWarning, stacklevel=3)
            return
        self.runtime_ok = False
        if strict_mode():
            raise RuntimeError(f"{self.label} HIP {what} failed and strict mode is enabled.") from exc
        if not self.warned:
            self.warned = True
            warnings.warn(
                f"[Qwen-Triton fallback] {self.label} HIP kernel unavailable "
                f"({exc.__class__.__name__}: {exc}). Using torch fallback.",
                RuntimeWarning,
                stacklevel=3,
            )

    def reset(self) -> None:
        self.runtime_ok = True
        self.warned = False
        self.unsupported_seen.clear()


def needs_grad(*tensors: torch.Tensor | None) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors)


def dense(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()
