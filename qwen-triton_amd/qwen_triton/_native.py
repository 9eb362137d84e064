"""ctypes binding of the gfx950 operator library ``libqwen_hip.so``.

The library exposes a plain C ABI (``include/qwen_hip.h``): device pointers,
int64 sizes/strides, a dtype code and the caller's HIP stream. This module
loads it once, declares every entry point's signature, maps non-zero return
codes to :class:`NativeError` carrying ``qh_last_error()``, and counts successful
calls per entry point so tests can prove that the HIP path (not a fallback) executed.
"""
from __future__ import annotations

import ctypes
import os
import re
from collections import Counter
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("QWEN_HIP_LIB", Path(__file__).resolve().parent / "_lib" / "libqwen_hip.so"))

F32, F16, BF16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_P = ctypes.c_void_p
_L = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

HEADER_PATH = Path(__file__).resolve().parents[2] / "include" / "qwen_hip.h"

_CT = {"p": _P, "l": _L, "i": _I, "f": _F}

_DECL_RE = re.compile(r"^\s*(int64_t|int|const char\s*\*)\s+(qh_\w+)\s*\(([^)]*)\)\s*;", re.M | re.S)


def _arg_code(decl: str) -> str:
    decl = decl.strip()
    if "*" in decl:
        return "p"
    base = decl.replace("const ", "").split()[0]
    return {"int64_t": "l", "int": "i", "float": "f", "int32_t": "i"}[base]


def parse_header(path: Path = HEADER_PATH) -> dict[str, tuple[str, str]]:
    """Map every `qh_*` declaration of the C header to (restype, argcodes)."""
    text = re.sub(r"/\*.*?\*/", "", path.read_text(), flags=re.S)
    sigs: dict[str, tuple[str, str]] = {}
    for ret, name, args in _DECL_RE.findall(text):
        ret = ret.replace(" ", "")
        rcode = {"int64_t": "l", "int": "i", "constchar*": "s"}[ret]
        args = args.strip()
        codes = "" if args in ("", "void") else "".join(_arg_code(a) for a in args.split(","))
        sigs[name] = (rcode, codes)
    return sigs


_SIGNATURES: dict[str, tuple[str, str]] = {}

CALLS: Counter = Counter()

_lib: ctypes.CDLL | None = None
_load_error: Exception | None = None
_load_attempted = False


class NativeError(RuntimeError):
    """A libqwen_hip entry point returned a non-zero status."""


class Unsupported(ValueError):
    """Inputs that are valid for the operator but outside what the HIP kernels take (a dtype, a head
    dimension, an alignment or layout). Raised before anything is launched; the operator wrappers run
    such a call on torch and keep using the kernels for later calls."""


class NativeUnsupported(NativeError, Unsupported):
    """The library rejected its arguments (QH_E_ARG / QH_E_DTYPE) before launching anything."""


_REJECTED = (1, 2)  # QH_E_ARG, QH_E_DTYPE: argument checks that run before any launch


def _bind(lib: ctypes.CDLL, name: str) -> None:
    restype, argtypes = _SIGNATURES[name]
    fn = getattr(lib, name)
    fn.restype = ctypes.c_char_p if restype == "s" else _CT[restype]
    fn.argtypes = [_CT[c] for c in argtypes]


def load() -> ctypes.CDLL | None:
    """Load the library once; returns None (and records the error) on failure."""
    global _lib, _load_error, _load_attempted
    if _lib is not None or _load_attempted:
        return _lib
    _load_attempted = True
    try:
        _SIGNATURES.update(parse_header())
        lib = ctypes.CDLL(str(LIB_PATH))
        for name in _SIGNATURES:
            _bind(lib, name)
        _lib = lib
    except Exception as exc:  # missing file, missing symbol, wrong arch
        _load_error = exc
        _lib = None
    return _lib


def available() -> bool:
    return load() is not None


def load_error() -> Exception | None:
    load()
    return _load_error


def lib() -> ctypes.CDLL:
    handle = load()
    if handle is None:
        raise RuntimeError(
            f"libqwen_hip.so could not be loaded from {LIB_PATH} ({_load_error!r}); "
            "build it with `python qwen-triton_amd/build.py`"
        )
    return handle


def version() -> str:
    return lib().qh_version().decode()


_FNS: dict[str, tuple] = {}


def call(name: str, *args) -> int:
    """Invoke an entry point; raise NativeError on a non-zero status."""
    entry = _FNS.get(name)
    if entry is None:
        handle = lib()
        entry = _FNS[name] = (getattr(handle, name), _SIGNATURES[name][0] == "i")
    fn, checked = entry
    rc = fn(*args)
    if checked and rc != 0:
        msg = lib().qh_last_error().decode(errors="replace")
        cls = NativeUnsupported if rc in _REJECTED else NativeError
        raise cls(f"{name} failed (status {rc}): {msg}")
    CALLS[name] += 1  # counts calls that returned success
    return rc


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise Unsupported(f"libqwen_hip supports float32/float16/bfloat16, got {dtype}") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device | None = None) -> int:
    """Raw handle of torch's current stream on ``device`` (the stream every kernel is enqueued on)."""
    if device is None:
        index = torch.cuda.current_device()
    else:
        index = device.index if isinstance(device, torch.device) else int(device)
        if index is None:
            index = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def require_device(*tensors: torch.Tensor | None) -> None:
    """Native kernels only take device tensors; anything else is a caller error."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise Unsupported("libqwen_hip kernels require GPU tensors")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)

