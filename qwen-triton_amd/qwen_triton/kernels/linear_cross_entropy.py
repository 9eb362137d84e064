"""Fused LM head + cross-entropy: ``cross_entropy(hidden @ weight.T, targets)`` without the logits.

The reference computes the LM head with ``triton_matmul`` (qwen_triton/kernels/matmul.py:130-200),
writing [N, V] logits, then ``triton_cross_entropy`` (qwen_triton/kernels/cross_entropy.py:55-226),
and lists the fused form as its next step (README.md:370). Here:

* forward: one tiled GEMM whose epilogue reduces each 256-column logit tile to per-row
  (max, sum of exp) partials and picks the target logit, then a fixed-order combine: the loss
  and the per-row logsumexp, with no [N, V] tensor;
* backward, one vocabulary chunk at a time: the chunk's logits are recomputed with an epilogue
  that writes their gradient ``(softmax - onehot) * g / n_valid`` ([N, chunk], the only large
  buffer), ``dW[chunk] = G^T X`` is written directly and ``dX += G W[chunk]`` accumulates in fp32
  over the chunks in order (deterministic).

Logits are rounded to the activation dtype before the softmax, as the unfused LM head writes them,
so results match ``triton_cross_entropy(triton_matmul(x, w), t)`` within fp32 summation order.
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, Unsupported, needs_grad

_GUARD = OpGuard("LinearCrossEntropy")

# vocabulary columns per backward chunk: the chunk's logit gradient ([N, chunk] in the activation
# dtype) is the only large temporary
CHUNK = 8192


def _torch_linear_cross_entropy(x, weight, targets, ignore_index: int = -100) -> torch.Tensor:
    logits = torch.nn.functional.linear(x, weight)
    return torch.nn.functional.cross_entropy(logits.float(), targets, ignore_index=ignore_index)


def _check(x: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor):
    _native.require_device(x, weight, targets)
    if x.dim() != 2 or weight.dim() != 2 or x.shape[1] != weight.shape[1]:
        raise Unsupported(f"linear cross-entropy expects x [N, H], weight [V, H]; got {tuple(x.shape)}, "
                          f"{tuple(weight.shape)}")
    if x.dtype != weight.dtype or x.dtype not in (torch.bfloat16, torch.float16):
        raise Unsupported("the fused LM head + cross-entropy kernels take bf16/fp16 x and weight of one dtype")
    if x.shape[1] % 8 or weight.shape[0] % 8:
        raise Unsupported("the fused LM head + cross-entropy kernels need H and V multiples of 8")
    if targets.numel() != x.shape[0]:
        raise Unsupported("targets must have one entry per row of x")


def _rows(t: torch.Tensor) -> torch.Tensor:
    return t if (t.stride(-1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0) else t.contiguous()


def linear_ce_forward(x, weight, targets, ignore_index: int):
    _check(x, weight, targets)
    x, w = _rows(x), _rows(weight)
    tg = targets.reshape(-1).contiguous().long()
    N, H = x.shape
    V = w.shape[0]
    dev = x.device
    lse = torch.empty(N, dtype=torch.float32, device=dev)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    nvalid = torch.empty(1, dtype=torch.float32, device=dev)
    ws = _native.workspace(_native.call("qh_lmce_workspace", N, V), dev)
    _native.call("qh_lmce_fwd", x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), tg.data_ptr(), N, V, H,
                 int(ignore_index), lse.data_ptr(), None, loss.data_ptr(), nvalid.data_ptr(), ws.data_ptr(),
                 ws.numel(), _native.dtype_code(x.dtype), _native.stream(dev))
    return loss, lse, nvalid, tg


def linear_ce_backward(x, weight, tg, lse, nvalid, grad_loss, ignore_index: int, need_x: bool, need_w: bool,
                       chunk: int | None = None):
    chunk = CHUNK if chunk is None else chunk
    x, w = _rows(x), _rows(weight)
    N, H = x.shape
    V = w.shape[0]
    dev = x.device
    code = _native.dtype_code(x.dtype)
    st = _native.stream(dev)
    g = grad_loss.reshape(1).to(torch.float32).contiguous()
    chunk = max(8, min(chunk, V) // 8 * 8)
    G = torch.empty((N, chunk), dtype=x.dtype, device=dev)
    dx32 = torch.zeros((N, H), dtype=torch.float32, device=dev) if need_x else None
    dw = torch.empty((V, H), dtype=weight.dtype, device=dev) if need_w else None
    from .matmul import gemm

    for v0 in range(0, V, chunk):
        vc = min(chunk, V - v0)
        _native.call("qh_lmce_grad", x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), tg.data_ptr(),
                     lse.data_ptr(), g.data_ptr(), nvalid.data_ptr(), N, v0, vc, H, int(ignore_index), G.data_ptr(),
                     G.stride(0), code, st)
        if need_w:  # dW[v0:v0+vc] = G^T X: A(m, k) = G[k, m], B(n, k) = X[k, n]
            gemm(True, True, vc, H, N, G, G.stride(0), x, x.stride(0), dw[v0:v0 + vc], H)
        if need_x:  # dX += G W[v0:v0+vc]: A = G [N, vc], B(n, k) = W[v0 + k, n]
            wc = w[v0:v0 + vc]
            _native.call("qh_gemm_acc", 0, 1, N, H, vc, G.data_ptr(), G.stride(0), wc.data_ptr(), wc.stride(0),
                         dx32.data_ptr(), H, code, st)
    return (dx32.to(x.dtype) if need_x else None), dw


class _LinearCrossEntropyFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, targets, ignore_index):
        loss, lse, nvalid, tg = linear_ce_forward(x, weight, targets, ignore_index)
        ctx.save_for_backward(x, weight, tg, lse, nvalid)
        ctx.ignore_index = ignore_index
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        x, weight, tg, lse, nvalid = ctx.saved_tensors
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        try:
            dx, dw = linear_ce_backward(x, weight, tg, lse, nvalid, grad_loss, ctx.ignore_index, need_x, need_w)
        except Exception as exc:
            _GUARD.failed(exc, "backward kernel")
            with torch.enable_grad():
                xx, ww = x.detach().requires_grad_(need_x), weight.detach().requires_grad_(need_w)
                ref = _torch_linear_cross_entropy(xx, ww, tg, ctx.ignore_index)
                grads = torch.autograd.grad(ref, [t for t in (xx, ww) if t.requires_grad], grad_loss)
            it = iter(grads)
            dx = next(it) if need_x else None
            dw = next(it) if need_w else None
        return dx, dw, None, None


def fused_linear_cross_entropy(x: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                               ignore_index: int = -100, use_triton: bool | None = None) -> torch.Tensor:
    """Mean cross-entropy of ``x @ weight.T`` against ``targets`` (fp32 scalar), as
    ``triton_cross_entropy(triton_matmul(x, weight), targets, ignore_index)`` computes it, with
    gradients for ``x`` and ``weight``; x [N, H], weight [V, H], targets [N]."""
    if not _GUARD.use_native(use_triton, x, weight, targets):
        return _torch_linear_cross_entropy(x, weight, targets, ignore_index)
    try:
        if needs_grad(x, weight):
            return _LinearCrossEntropyFunction.apply(x, weight, targets, ignore_index)
        return linear_ce_forward(x, weight, targets, ignore_index)[0]
    except Exception as exc:
        _GUARD.failed(exc)
        return _torch_linear_cross_entropy(x, weight, targets, ignore_index)
