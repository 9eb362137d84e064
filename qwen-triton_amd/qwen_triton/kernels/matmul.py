"""Linear layer GEMM ``y = x @ W^T (+ b)`` and its backward on the HIP library.

Reference: qwen_triton/kernels/matmul.py:35-255 (torch fallbacks :35-49, tile
kernel :64-97, bias/row-sum kernels :100-127, forward :130-155, backward
:158-200, autograd :203-232, public op :235-255).

The three products run on one MFMA kernel with operand-view flags, so neither
``W.T`` (reference :140) nor ``grad.T`` (:184) is ever materialised:
forward ``x W^T`` (NT), input grad ``dy W`` (B transposed view) and weight grad
``dy^T x`` (both operands transposed views).
"""
from __future__ import annotations

import ctypes
import os

import torch

from .. import _native
from ._common import OpGuard, needs_grad, Unsupported

_GUARD = OpGuard("Matmul")

# Inference products behind an RMSNorm (q/k/v, gate/up) read a copy of their weights with the norm
# weight folded in (``_folded_group``): one extra copy of those weights per model, about 0.59 GB at
# Qwen3-0.6B (28 layers x (8 + 12) MB), kept on the norm weight until ``release_folded_weights``.
# With the switch off (or QWEN_TRITON_FOLD_NORM=0) no copy is made: the launch scales the weight
# fragments itself (``qh_gemm_multi_ex``, same bits for more than 4 rows) where its shape fits one
# load chunk per workgroup, and the layer otherwise runs the separate norm and products.
FOLD_NORM_WEIGHTS = os.environ.get("QWEN_TRITON_FOLD_NORM", "1") != "0"


def _torch_matmul(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    return torch.nn.functional.linear(x, weight, bias)


def _torch_matmul_backward(x, weight, grad_output, needs_bias_grad: bool):
    grad_x = grad_output @ weight
    g2 = grad_output.reshape(-1, grad_output.shape[-1])
    grad_weight = g2.T @ x.reshape(-1, x.shape[-1])
    grad_bias = g2.sum(0) if needs_bias_grad else None
    return grad_x, grad_weight, grad_bias


def _rows(t: torch.Tensor, cols: int) -> torch.Tensor:
    """2-D row-major view [rows, cols] with unit column stride (copies only if needed)."""
    t2 = t.reshape(-1, cols)
    if t2.stride(1) != 1 or (t2.shape[0] > 1 and t2.stride(0) < cols):
        t2 = t2.contiguous()
    return t2


def gemm(trans_a: bool, trans_b: bool, M: int, N: int, K: int, a: torch.Tensor, lda: int, b: torch.Tensor, ldb: int,
         out: torch.Tensor, ldc: int, bias: torch.Tensor | None = None) -> torch.Tensor:
    """Raw library GEMM: out[M,N] = A(M,K) . B(N,K)^T (+ bias) with operand views.

    Products with few output tiles and a long K (weight gradients) get a workspace so the
    library can split K."""
    code = _native.dtype_code(a.dtype)
    args = (int(trans_a), int(trans_b), M, N, K, a.data_ptr(), lda, b.data_ptr(), ldb, out.data_ptr(), ldc,
            None if bias is None else bias.data_ptr(), code, _native.dtype_code(out.dtype))
    if K >= 2048 and M >= 256 and N >= 256 and M * N < 128 * 65536:
        nbytes = _native.call("qh_gemm_workspace", M, N, K, code)
        if nbytes:
            ws = _native.workspace(nbytes, a.device)
            _native.call("qh_gemm_ws", *args, ws.data_ptr(), ws.numel(), _native.stream(a.device))
            return out
    _native.call("qh_gemm", *args, _native.stream(a.device))
    return out


def linear_group_ok(x: torch.Tensor, weights: list[torch.Tensor]) -> bool:
    """True when ``linear_group`` can serve these operands (decode-sized, k-contiguous, aligned)."""
    if not (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and _native.available()):
        return False
    k = x.shape[-1]
    if k % 8 or x.numel() // max(k, 1) > 128 or not 1 <= len(weights) <= 4:
        return False
    return all(w.dtype == x.dtype and w.is_cuda and w.dim() == 2 and w.shape[1] == k and w.stride(1) == 1
               and w.stride(0) % 8 == 0 and w.data_ptr() % 16 == 0 for w in weights)


_PLANS: dict[tuple, tuple] = {}


def _group_plan(weights: list[torch.Tensor], biases: list[torch.Tensor | None] | None) -> tuple:
    """Host argument arrays of the weight side of a grouped launch (pointer, row stride and rows of
    each weight, bias pointers), built once per set of weight and bias tensors."""
    n = len(weights)
    biases = biases or [None] * n
    key = tuple((w.data_ptr(), w.shape[0], w.stride(0)) for w in weights) + tuple(
        None if b is None else (b.data_ptr(), b.stride(0)) for b in biases)
    plan = _PLANS.get(key)
    if plan is None:
        if len(_PLANS) > 4096:
            _PLANS.clear()
        arr_p = ctypes.c_void_p * n
        arr_l = ctypes.c_int64 * n
        bptr = arr_p(*(w.data_ptr() for w in weights))
        ldb = arr_l(*(w.stride(0) for w in weights))
        nn_ = arr_l(*(w.shape[0] for w in weights))
        if any(b is not None for b in biases):
            if any(b is not None and b.stride(0) != 1 for b in biases):
                raise ValueError("linear_group: biases must be contiguous")
            bias_arr = arr_p(*(None if b is None else b.data_ptr() for b in biases))
            plan = (bptr, ldb, nn_, ctypes.addressof(bias_arr), bias_arr)
        else:
            plan = (bptr, ldb, nn_, None)
        _PLANS[key] = plan
    return plan


def linear_group_norm_ok(x: torch.Tensor, weights: list[torch.Tensor], norm_weight: torch.Tensor,
                         gated: bool = False) -> bool:
    """True when ``linear_group(..., norm=...)`` can normalise the rows of ``x`` inside the launch."""
    if not linear_group_ok(x, weights):
        return False
    k = x.shape[-1]
    if not (norm_weight.is_cuda and norm_weight.dim() == 1 and norm_weight.shape[0] == k
            and norm_weight.is_contiguous() and norm_weight.dtype == x.dtype):
        return False
    if gated and not (len(weights) == 2 and weights[0].shape[0] == weights[1].shape[0]):
        return False
    if FOLD_NORM_WEIGHTS:
        return True
    ns = (ctypes.c_int64 * len(weights))(*(w.shape[0] for w in weights))
    return bool(_native.call("qh_gemm_multi_norm_fits", x.numel() // k, k, int(gated), len(weights),
                             ctypes.addressof(ns)))


def release_folded_weights(module: torch.nn.Module) -> int:
    """Free the norm-folded weight copies made for ``module``'s inference products (they are made
    again on the next such call while ``FOLD_NORM_WEIGHTS`` is on). Returns the bytes released.
    Captured graphs that read the copies keep them alive until the graphs are dropped."""
    freed = 0
    for t in list(module.parameters()) + list(module.buffers()):
        store = t.__dict__.pop("_qh_folded", None)
        for _, folded, fb in (store or {}).values():
            freed += sum(w.numel() * w.element_size() for w in folded)
            freed += sum(b.numel() * b.element_size() for b in (fb or []) if b is not None)
    return freed


def folded_weight_tensors(module: torch.nn.Module) -> list[torch.Tensor]:
    """The norm-folded weight copies currently kept for ``module`` (see ``_folded_group``)."""
    out = []
    for t in list(module.parameters()) + list(module.buffers()):
        for _, folded, fb in getattr(t, "_qh_folded", {}).values():
            out.extend(folded)
            out.extend(b for b in (fb or []) if b is not None)
    return out


def _folded_group(weights: list[torch.Tensor], biases: list[torch.Tensor | None] | None, norm_weight: torch.Tensor,
                  one_plus: bool, concat: bool) -> tuple[list[torch.Tensor], list[torch.Tensor | None] | None]:
    """The weights with the RMSNorm weight folded in, ``round(W * (w + one_plus))`` per column as the
    in-kernel norm rounds its weight operand (fp32 product, one rounding to the dtype), made once and
    kept on the norm weight; rebuilt when any of the tensors is modified (version counters). With
    ``concat`` the products are stacked into one weight (and bias) so that one product serves them."""
    sig = (tuple((w.data_ptr(), tuple(w.shape), w.stride(0)) for w in weights), bool(one_plus), bool(concat),
           None if biases is None else tuple(None if b is None else b.data_ptr() for b in biases))
    versions = (tuple(w._version for w in weights), norm_weight._version, norm_weight.data_ptr(),
                None if biases is None else tuple(None if b is None else b._version for b in biases))
    store = getattr(norm_weight, "_qh_folded", None)
    if store is None:
        store = {}
        norm_weight._qh_folded = store
    hit = store.get(sig)
    if hit is not None and hit[0] == versions:
        return hit[1], hit[2]
    with torch.no_grad():
        scale = norm_weight.float() + (1.0 if one_plus else 0.0)
        folded = [(w.float() * scale).to(w.dtype) for w in weights]
        fb = biases
        if concat:
            folded = [torch.cat(folded)]
            if biases is not None and all(b is not None for b in biases):
                fb = [torch.cat([b.reshape(-1) for b in biases])]
            else:
                fb = None
    if len(store) > 8:
        store.clear()
    store[sig] = (versions, folded, fb)
    return folded, fb


def linear_group(x: torch.Tensor, weights: list[torch.Tensor], biases: list[torch.Tensor | None] | None = None,
                 gated: bool = False, norm: tuple[torch.Tensor, float, bool] | None = None,
                 residual: list[torch.Tensor | None] | None = None):
    """One launch for ``x @ W_i.T (+ b_i)`` over products that share ``x`` (M <= 128, no autograd).

    Returns the list of outputs, or ``silu(x @ W_0.T) * (x @ W_1.T)`` when ``gated``; each
    product is computed and rounded exactly as ``triton_matmul`` would.

    ``norm = (weight, eps, one_plus)``: ``x`` holds RMSNorm inputs and the products use
    ``rmsnorm(x)``: the norm weight is folded into the weights once (``round(W * (weight +
    one_plus))``, kept with the norm weight, see ``_folded_group``) and each output row is scaled
    by ``rsqrt(mean(x^2) + eps)`` after the sum over K, so the one rounding of the normalised
    operand sits in the weight operand, before the row factor (check ``linear_group_norm_ok``
    first; the weight has the activation dtype). Non-gated groups run as one product over the
    stacked weights and return column views of its output. ``residual[i]`` (same shape as output
    i): output i is ``residual_add(x @ W_i.T (+ b_i), residual[i])``, rounded as the two kernels
    round.
    """
    k = x.shape[-1]
    x2 = _rows(x, k)
    m = x2.shape[0]
    if norm is not None:
        if residual is not None:
            raise ValueError("linear_group: norm and residual do not combine")
        return _linear_group_rms(x, x2, weights, biases, gated, norm)
    n = len(weights)
    plan = _group_plan(weights, biases)
    outs = [torch.empty((m, w.shape[0]), dtype=x.dtype, device=x.device) for w in (weights[:1] if gated else weights)]
    arr_p = ctypes.c_void_p * n
    arr_l = ctypes.c_int64 * n
    cptr = arr_p(*([o.data_ptr() for o in outs] + [None] * (n - len(outs))))
    ldc = arr_l(*([o.stride(0) for o in outs] + [0] * (n - len(outs))))
    bptr, ldb, nn_, bias_addr = plan[:4]  # `plan` keeps the bias array alive
    if norm is None and residual is None:
        _native.call("qh_gemm_multi", m, k, x2.data_ptr(), x2.stride(0), n, ctypes.addressof(bptr),
                     ctypes.addressof(ldb), ctypes.addressof(nn_), ctypes.addressof(cptr), ctypes.addressof(ldc),
                     bias_addr, int(gated), _native.dtype_code(x.dtype), _native.stream(x.device))
    else:
        res_arr = ldr = None
        if residual is not None:
            if gated or len(residual) != n:
                raise ValueError("linear_group: residual needs one entry per (non-gated) product")
            rs = []
            for r, o in zip(residual, outs):
                if r is None:
                    rs.append(None)
                    continue
                r2 = _rows(r, o.shape[1])
                if r2.shape != o.shape or r2.dtype != x.dtype or not r2.is_cuda:
                    raise ValueError(f"linear_group: residual {tuple(r.shape)} does not match output {tuple(o.shape)}")
                rs.append(r2)
            res_arr = arr_p(*(None if r is None else r.data_ptr() for r in rs))
            ldr = arr_l(*(0 if r is None else r.stride(0) for r in rs))
        _native.call("qh_gemm_multi_ex", m, k, x2.data_ptr(), x2.stride(0), n, ctypes.addressof(bptr),
                     ctypes.addressof(ldb), ctypes.addressof(nn_), ctypes.addressof(cptr), ctypes.addressof(ldc),
                     bias_addr, ctypes.addressof(res_arr) if res_arr is not None else None,
                     ctypes.addressof(ldr) if ldr is not None else None, int(gated), None, 0, 0.0, 0,
                     _native.dtype_code(x.dtype), _native.stream(x.device))
    lead = x.shape[:-1]
    outs = [o.view(*lead, o.shape[1]) for o in outs]
    return outs[0] if gated else outs


def _linear_group_rms(x, x2, weights, biases, gated, norm):
    """``linear_group(..., norm=...)``: folded weights, the row factor applied in the launch
    (``qh_gemm_multi_rms``)."""
    nw, eps, one_plus = norm
    k, m = x2.shape[1], x2.shape[0]
    if not FOLD_NORM_WEIGHTS:
        return _linear_group_norm_in_kernel(x, x2, weights, biases, gated, norm)
    concat = not gated and len(weights) > 1
    fw, fb = _folded_group(weights, biases, nw, one_plus, concat)
    n = len(fw)
    bptr, ldb, nn_, bias_addr = _group_plan(fw, fb)[:4]
    outs = [torch.empty((m, w.shape[0]), dtype=x.dtype, device=x.device) for w in (fw[:1] if gated else fw)]
    arr_p = ctypes.c_void_p * n
    arr_l = ctypes.c_int64 * n
    cptr = arr_p(*([o.data_ptr() for o in outs] + [None] * (n - len(outs))))
    ldc = arr_l(*([o.stride(0) for o in outs] + [0] * (n - len(outs))))
    _native.call("qh_gemm_multi_rms", m, k, x2.data_ptr(), x2.stride(0), n, ctypes.addressof(bptr),
                 ctypes.addressof(ldb), ctypes.addressof(nn_), ctypes.addressof(cptr), ctypes.addressof(ldc),
                 bias_addr, int(gated), float(eps), _native.dtype_code(x.dtype), _native.stream(x.device))
    lead = x.shape[:-1]
    if gated:
        return outs[0].view(*lead, outs[0].shape[1])
    if concat:
        cols, c0 = [], 0
        for w in weights:
            cols.append(outs[0][:, c0:c0 + w.shape[0]].view(*lead, w.shape[0]))
            c0 += w.shape[0]
        return cols
    return [outs[0].view(*lead, outs[0].shape[1])]


def _linear_group_norm_in_kernel(x, x2, weights, biases, gated, norm):
    """``linear_group(..., norm=...)`` without a folded copy: the launch scales the weight
    fragments by the norm weight itself (``qh_gemm_multi_ex``)."""
    nw, eps, one_plus = norm
    k, m = x2.shape[1], x2.shape[0]
    n = len(weights)
    bptr, ldb, nn_, bias_addr = _group_plan(weights, biases)[:4]
    outs = [torch.empty((m, w.shape[0]), dtype=x.dtype, device=x.device) for w in (weights[:1] if gated else weights)]
    arr_p = ctypes.c_void_p * n
    arr_l = ctypes.c_int64 * n
    cptr = arr_p(*([o.data_ptr() for o in outs] + [None] * (n - len(outs))))
    ldc = arr_l(*([o.stride(0) for o in outs] + [0] * (n - len(outs))))
    code = _native.dtype_code(x.dtype)
    _native.call("qh_gemm_multi_ex", m, k, x2.data_ptr(), x2.stride(0), n, ctypes.addressof(bptr),
                 ctypes.addressof(ldb), ctypes.addressof(nn_), ctypes.addressof(cptr), ctypes.addressof(ldc),
                 bias_addr, None, None, int(gated), nw.data_ptr(), code, float(eps), int(bool(one_plus)), code,
                 _native.stream(x.device))
    lead = x.shape[:-1]
    outs = [o.view(*lead, o.shape[1]) for o in outs]
    return outs[0] if gated else outs


def _native_matmul_forward(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    _native.require_device(x, weight, bias)
    if x.dtype != weight.dtype or (bias is not None and bias.dtype != weight.dtype):
        raise Unsupported("matmul kernel needs x, weight and bias of one dtype")
    N, K = weight.shape
    if x.shape[-1] != K:
        raise Unsupported(f"matmul shape mismatch: x {tuple(x.shape)} weight {tuple(weight.shape)}")
    x2 = _rows(x, K)
    w = weight if weight.stride(1) == 1 else weight.contiguous()
    b = None if bias is None else bias.contiguous()
    M = x2.shape[0]
    out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    gemm(False, False, M, N, K, x2, x2.stride(0), w, w.stride(0), out, N, b)
    return out.view(*x.shape[:-1], N)


def _native_matmul_backward(x, weight, grad_output, need_x: bool, need_w: bool, need_b: bool):
    N, K = weight.shape
    g2 = _rows(grad_output.to(weight.dtype), N)
    M = g2.shape[0]
    grad_x = grad_w = grad_b = None
    if need_x:
        w = weight if weight.stride(1) == 1 else weight.contiguous()
        grad_x = torch.empty((M, K), dtype=x.dtype, device=x.device)
        gemm(False, True, M, K, N, g2, g2.stride(0), w, w.stride(0), grad_x, K)
        grad_x = grad_x.view(x.shape)
    if need_w:
        x2 = _rows(x, K)
        grad_w = torch.empty((N, K), dtype=weight.dtype, device=weight.device)
        gemm(True, True, N, K, M, g2, g2.stride(0), x2, x2.stride(0), grad_w, K)
    if need_b:
        grad_b = torch.empty((N,), dtype=weight.dtype, device=weight.device)
        _native.call("qh_colsum", g2.data_ptr(), g2.stride(0), M, N, grad_b.data_ptr(),
                     _native.dtype_code(g2.dtype), _native.dtype_code(grad_b.dtype), _native.stream(g2.device))
    return grad_x, grad_w, grad_b


class _MatmulFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return _native_matmul_forward(x, weight, bias)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        x, weight = ctx.saved_tensors
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        need_b = ctx.has_bias and ctx.needs_input_grad[2]
        try:
            return _native_matmul_backward(x, weight, grad_output, need_x, need_w, need_b)
        except Exception as exc:
            _GUARD.failed(exc, "backward kernel")
            gx, gw, gb = _torch_matmul_backward(x, weight, grad_output, need_b)
            return gx, gw, gb


def triton_matmul(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    use_triton: bool | None = None,
) -> torch.Tensor:
    if not _GUARD.use_native(use_triton, x, weight):
        return _torch_matmul(x, weight, bias)
    try:
        if needs_grad(x, weight, bias):
            return _MatmulFunction.apply(x, weight, bias)
        return _native_matmul_forward(x, weight, bias)
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_matmul(x, weight, bias)
