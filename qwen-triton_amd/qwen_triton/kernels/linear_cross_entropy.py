"""Fused LM head + cross-entropy: ``cross_entropy(hidden @ weight.T, targets)`` without [N, V] logits.

The reference computes the LM head with ``triton_matmul`` (qwen_triton/kernels/matmul.py:130-200),
writing [N, V] logits, then ``triton_cross_entropy`` (qwen_triton/kernels/cross_entropy.py:55-226),
and lists the fused form as its next step (README.md:370). Here:

* without gradients: one tiled GEMM whose epilogue reduces each 256-column logit tile to per-row
  (max, sum of exp) partials and picks the target logit, then a fixed-order combine: the loss and
  the per-row logsumexp, with no [N, V] tensor at all;
* with gradients, everything happens in the forward, one block of rows at a time
  (each logit is computed once): the block's logits Z (the only [rows, V] buffer) come out of a
  GEMM whose epilogue also forms per-64-column (max, sum of exp) partials, so the block's
  logsumexp needs no pass over Z; Z is turned into the logit gradient ``(softmax - onehot) /
  n_valid`` in place, then ``dX[block] = G W`` and ``dW += G^T X[block]`` (fp32, blocks added in
  order: deterministic). The backward only multiplies the fp32 gradients by the upstream gradient
  of the loss and rounds them.

Logits are rounded to the activation dtype before the softmax, as the unfused LM head writes them,
so results match ``triton_cross_entropy(triton_matmul(x, w), t)`` within fp32 summation order (and
exactly the unfused gradient values G when the upstream gradient is 1).
"""
from __future__ import annotations

import torch

from .. import _native
from ._common import OpGuard, Unsupported, needs_grad

_GUARD = OpGuard("LinearCrossEntropy")

# Rows per block of the training path: as many as keep the block's logits / logit gradient
# ([rows, V] in the activation dtype) within ROW_BLOCK_BYTES (rounded down to 256 rows, the GEMM
# tile), the largest temporary besides the fp32 dW; fewer blocks mean fewer fp32 accumulations of
# dW (at 16384 x 151936: three blocks of at most 5632 rows, 1.71 GB). ROW_CHUNK, when set, fixes
# the row count instead.
ROW_BLOCK_BYTES = 1792 << 20
ROW_CHUNK: int | None = None


def _block_rows(N: int, V: int, itemsize: int) -> int:
    if ROW_CHUNK is not None:
        return int(ROW_CHUNK)
    cap = max(256, ROW_BLOCK_BYTES // max(1, V * itemsize) // 256 * 256)
    nblk = max(1, -(-N // cap))
    if nblk == 1:
        return N
    per = -(-N // nblk)
    return -(-per // 256) * 256


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


def linear_ce_train(x, weight, targets, ignore_index: int, need_x: bool, need_w: bool, rows: int | None = None):
    """Loss (fp32 scalar) and the gradients of x and weight for an upstream gradient of 1, as fp32
    tensors (None where not needed), one block of ``rows`` rows at a time."""
    _check(x, weight, targets)
    x, w = _rows(x), _rows(weight)
    tg = targets.reshape(-1).contiguous().long()
    N, H = x.shape
    V = w.shape[0]
    dev = x.device
    code = _native.dtype_code(x.dtype)
    st = _native.stream(dev)
    rows = _block_rows(N, V, x.element_size()) if rows is None else int(rows)
    rows = max(1, min(rows, N)) if N else 1
    from .matmul import gemm

    lse = torch.empty(N, dtype=torch.float32, device=dev)
    loss_rows = torch.empty(N, dtype=torch.float32, device=dev)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    nvalid = torch.empty(1, dtype=torch.float32, device=dev)
    one = torch.ones(1, dtype=torch.float32, device=dev)
    dx32 = torch.empty((N, H), dtype=torch.float32, device=dev) if need_x else None
    dw32 = torch.empty((V, H), dtype=torch.float32, device=dev) if need_w else None
    if need_w and N == 0:
        dw32.zero_()
    Z = torch.empty((rows, V), dtype=x.dtype, device=dev)
    ws = _native.workspace(_native.call("qh_lmce_rows_workspace", rows, V), dev)
    _native.call("qh_lmce_count", tg.data_ptr(), N, int(ignore_index), nvalid.data_ptr(), st)
    for r0 in range(0, N, rows):
        rc = min(rows, N - r0)
        xc, tc = x[r0:r0 + rc], tg[r0:r0 + rc]
        _native.call("qh_lmce_rows_fwd", xc.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), tc.data_ptr(), rc, V,
                     H, int(ignore_index), Z.data_ptr(), Z.stride(0), lse[r0:].data_ptr(), loss_rows[r0:].data_ptr(),
                     ws.data_ptr(), ws.numel(), code, st)
        if not (need_x or need_w):
            continue
        # logit gradient of the block, in place: (softmax - onehot) / n_valid
        _native.call("qh_ce_bwd", Z.data_ptr(), Z.stride(0), tc.data_ptr(), lse[r0:].data_ptr(), one.data_ptr(),
                     nvalid.data_ptr(), Z.data_ptr(), Z.stride(0), rc, V, int(ignore_index), code, st)
        G = Z[:rc]
        if need_x:  # dX[block] = G W: B(n, k) = W[k, n]
            gemm(False, True, rc, H, V, G, G.stride(0), w, w.stride(0), dx32[r0:r0 + rc], H)
        if need_w:  # dW (+)= G^T X[block]: A(m, k) = G[k, m], B(n, k) = X[k, n]
            if r0 == 0:
                gemm(True, True, V, H, rc, G, G.stride(0), xc, x.stride(0), dw32, H)
            else:
                _native.call("qh_gemm_acc", 1, 1, V, H, rc, G.data_ptr(), G.stride(0), xc.data_ptr(), x.stride(0),
                             dw32.data_ptr(), H, code, st)
    _native.call("qh_lmce_finish", loss_rows.data_ptr(), tg.data_ptr(), N, int(ignore_index), loss.data_ptr(),
                 nvalid.data_ptr(), st)
    return loss, dx32, dw32


def _scaled(g32: torch.Tensor | None, g: torch.Tensor, dtype: torch.dtype) -> torch.Tensor | None:
    if g32 is None:
        return None
    out = torch.empty(g32.shape, dtype=dtype, device=g32.device)
    _native.call("qh_scale_cast", g32.data_ptr(), out.data_ptr(), g32.numel(), g.data_ptr(),
                 _native.dtype_code(dtype), _native.stream(g32.device))
    return out


class _LinearCrossEntropyFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, targets, ignore_index):
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        loss, dx32, dw32 = linear_ce_train(x, weight, targets, ignore_index, need_x, need_w)
        ctx.save_for_backward(dx32, dw32)
        ctx.dtypes = (x.dtype, weight.dtype)
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        dx32, dw32 = ctx.saved_tensors
        g = grad_loss.reshape(1).to(torch.float32).contiguous()
        dx = _scaled(dx32, g, ctx.dtypes[0])
        dw = _scaled(dw32, g, ctx.dtypes[1])
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
