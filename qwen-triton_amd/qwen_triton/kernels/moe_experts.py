"""Expert computation of the sparse MoE block as dispatch + grouped GEMM + combine.

Reference: the per-expert loop of ``QwenSparseMoeBlock.forward``
(qwen_triton/modules/moe.py:45-51): one-hot/nonzero/where to find each
expert's tokens, the expert SwiGLU MLP on them, scaling by the routing weight
and ``triton_index_add`` into a zero tensor in ascending expert order.

Here the routed (token, slot) pairs are sorted by expert once
(``qh_moe_dispatch``), both expert GEMMs run as one grouped launch each over
all experts, and ``qh_moe_combine`` sums each token's expert rows in ascending
expert order with the reference's bf16 rounding after every add. No host
synchronisation; deterministic. With many routed rows per expert the forward
runs on the 256x256 tile kernels (the training forward below, without keeping
G and U); sparser routings use ``qh_moe_gemm`` (128-row tiles, gate/up with the
token gather and SiLU-mul fused, down with the routing-weight scaling fused).
Both round at the same points.

Training (autograd on) runs ``GroupedExperts``: the same dispatch (with 256-row
tiles), a gather of the routed rows, grouped GEMMs on the 256x256 tile kernel
(gate/up writing G, U and H = silu(G) U; down writing the unscaled expert
output D) and the combine with the routing-weight multiply fused. Its backward
mirrors the reference loop's autograd graph: the routing-weight multiply
(dD, d_weights), the down projection's input gradient with the SiLU-mul
backward fused (dG, dU), the gate/up input gradient (one K = 2I product),
the ordered combine of the routed rows' gradients, and the expert weight
gradients as grouped products that reduce over each expert's rows.
"""
from __future__ import annotations

import torch

from .. import _native

TILE_M = 128
MOE_GATED, MOE_SCALED = 0, 1


def moe_experts_forward(flat: torch.Tensor, routing_weights: torch.Tensor, selected: torch.Tensor,
                        gate_up_table: torch.Tensor, down_table: torch.Tensor, n_experts: int,
                        intermediate: int, weight_row_stride: tuple[int, int]) -> torch.Tensor:
    """flat [T, H]; routing_weights [T, k] (flat's dtype); selected [T, k] int64; tables: device int64
    pointer arrays (gate_e, up_e interleaved / down_e); weight_row_stride = (gate/up row stride, down row stride)."""
    _native.require_device(flat, routing_weights, selected)
    t, hidden = flat.shape
    if grouped_training_ok(hidden, intermediate) and t * selected.shape[1] >= TILE_FORWARD_MIN_ROWS * n_experts:
        return _tile_forward(flat, routing_weights, selected, gate_up_table, down_table, n_experts, intermediate,
                             weight_row_stride[0], weight_row_stride[1], False)[0]
    k = selected.shape[1]
    r = t * k
    dev, dt = flat.device, flat.dtype
    code = _native.dtype_code(dt)
    st = _native.stream(dev)
    sel = selected.contiguous()
    w = routing_weights.to(dt).contiguous()
    ws = _native.workspace(_native.call("qh_moe_dispatch_workspace", t, k, n_experts), dev)
    rows = torch.empty(r, dtype=torch.int32, device=dev)
    wsorted = torch.empty(r, dtype=dt, device=dev)
    inv = torch.empty(r, dtype=torch.int32, device=dev)
    seg = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    toff = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    _native.call("qh_moe_dispatch", sel.data_ptr(), w.data_ptr(), t, k, n_experts, TILE_M, ws.data_ptr(), ws.numel(),
                 rows.data_ptr(), wsorted.data_ptr(), inv.data_ptr(), seg.data_ptr(), toff.data_ptr(), code, st)
    x = flat if flat.stride(1) == 1 and flat.stride(0) % 8 == 0 else flat.contiguous()
    h = torch.empty((r, intermediate), dtype=dt, device=dev)
    _native.call("qh_moe_gemm", MOE_GATED, x.data_ptr(), x.stride(0), rows.data_ptr(), gate_up_table.data_ptr(),
                 weight_row_stride[0], h.data_ptr(), intermediate, None, seg.data_ptr(), toff.data_ptr(), r,
                 n_experts, intermediate, hidden, code, st)
    y = torch.empty((r, hidden), dtype=dt, device=dev)
    _native.call("qh_moe_gemm", MOE_SCALED, h.data_ptr(), intermediate, None, down_table.data_ptr(),
                 weight_row_stride[1], y.data_ptr(), hidden, wsorted.data_ptr(), seg.data_ptr(), toff.data_ptr(), r,
                 n_experts, hidden, intermediate, code, st)
    out = torch.empty((t, hidden), dtype=dt, device=dev)
    _native.call("qh_moe_combine", y.data_ptr(), hidden, inv.data_ptr(), sel.data_ptr(), None, t, k, n_experts,
                 out.data_ptr(), hidden, code, st)
    return out


TRAIN_TILE_M = 256
# With at least this many routed rows per expert on average, the inference forward runs on the
# 256x256 tile kernels (the training forward's; measured 1.7x faster at config 4's 1024 rows per
# expert); sparser routings keep the 128-row grouped kernel with its fused gather.
TILE_FORWARD_MIN_ROWS = 128


def grouped_training_ok(hidden: int, intermediate: int) -> bool:
    """Shapes the 256x256 tile kernels take (the feature dimensions tile evenly)."""
    return intermediate % 128 == 0 and hidden % 8 == 0


def _tile_forward(flat, routing_weights, selected, gu_table, dn_table, n_experts, intermediate, ldw_gu, ldw_dn,
                  keep_gu: bool):
    """Expert forward on the 256x256 tile kernels: dispatch (256-row tiles), gate/up with SiLU-mul
    (for training on a gathered copy of the routed rows, which the weight gradients read, with G and
    U written; for inference gathering the token rows itself), down (unscaled D) and the combine
    with the routing-weight multiply. Returns out and the tensors the backward uses."""
    t, hidden = flat.shape
    k = selected.shape[1]
    r = t * k
    dev, dt = flat.device, flat.dtype
    code = _native.dtype_code(dt)
    st = _native.stream(dev)
    sel = selected.contiguous()
    w = routing_weights.to(dt).contiguous()
    ws = _native.workspace(_native.call("qh_moe_dispatch_workspace", t, k, n_experts), dev)
    rows = torch.empty(r, dtype=torch.int32, device=dev)
    wsorted = torch.empty(r, dtype=dt, device=dev)
    inv = torch.empty(r, dtype=torch.int32, device=dev)
    seg = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    toff = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    _native.call("qh_moe_dispatch", sel.data_ptr(), w.data_ptr(), t, k, n_experts, TRAIN_TILE_M, ws.data_ptr(),
                 ws.numel(), rows.data_ptr(), wsorted.data_ptr(), inv.data_ptr(), seg.data_ptr(), toff.data_ptr(),
                 code, st)
    x = flat.contiguous()
    if keep_gu:  # the backward's weight gradients read the routed rows in sorted order
        xs = torch.empty((r, hidden), dtype=dt, device=dev)
        _native.call("qh_moe_gather", x.data_ptr(), hidden, rows.data_ptr(), r, hidden, xs.data_ptr(), hidden, code,
                     st)
        a, a_rows = xs, None
    else:  # inference: gate/up gathers the token rows itself
        xs, a, a_rows = None, x, rows.data_ptr()
    g = torch.empty((r, intermediate), dtype=dt, device=dev) if keep_gu else None
    u = torch.empty_like(g) if keep_gu else None
    h = torch.empty((r, intermediate), dtype=dt, device=dev)
    _native.call("qh_moe_up", a.data_ptr(), hidden, a_rows, r, hidden, gu_table.data_ptr(), ldw_gu, intermediate,
                 seg.data_ptr(), toff.data_ptr(), n_experts, None if g is None else g.data_ptr(),
                 None if u is None else u.data_ptr(), h.data_ptr(), intermediate, code, st)
    d = torch.empty((r, hidden), dtype=dt, device=dev)
    _native.call("qh_moe_down", h.data_ptr(), intermediate, r, intermediate, dn_table.data_ptr(), ldw_dn, hidden,
                 seg.data_ptr(), toff.data_ptr(), n_experts, d.data_ptr(), hidden, None, code, st)
    out = torch.empty((t, hidden), dtype=dt, device=dev)
    _native.call("qh_moe_combine", d.data_ptr(), hidden, inv.data_ptr(), sel.data_ptr(), w.data_ptr(), t, k,
                 n_experts, out.data_ptr(), hidden, code, st)
    return out, (w, sel, inv, seg, toff, xs, g, u, h, d)


class GroupedExperts(torch.autograd.Function):
    """Experts of the sparse MoE block with the reference loop's gradients.

    Inputs: flat [T, H], routing_weights [T, k] (flat's dtype), selected [T, k]
    int64, the device pointer tables (gate/up interleaved, down), the sizes,
    then the 3E expert weight tensors (gate_0, up_0, down_0, gate_1, ...) so
    autograd routes their gradients.
    """

    @staticmethod
    def forward(ctx, flat, routing_weights, selected, gu_table, dn_table, n_experts, intermediate, ldw_gu, ldw_dn,
                *weights):
        _native.require_device(flat, routing_weights, selected)
        t, hidden = flat.shape
        k = selected.shape[1]
        out, (w, sel, inv, seg, toff, xs, g, u, h, d) = _tile_forward(
            flat, routing_weights, selected, gu_table, dn_table, n_experts, intermediate, ldw_gu, ldw_dn, True)
        ctx.save_for_backward(w, sel, inv, seg, toff, xs, g, u, h, d, gu_table, dn_table)
        ctx.sizes = (t, k, hidden, intermediate, n_experts, ldw_gu, ldw_dn)
        ctx.weight_meta = [(wt.shape, wt.dtype) for wt in weights]
        ctx.rw_dtype = routing_weights.dtype
        return out

    @staticmethod
    def backward(ctx, dout):
        w, sel, inv, seg, toff, xs, g, u, h, d, gu_table, dn_table = ctx.saved_tensors
        t, k, hidden, inter, n_experts, ldw_gu, ldw_dn = ctx.sizes
        r = t * k
        dev, dt = xs.device, xs.dtype
        code = _native.dtype_code(dt)
        st = _native.stream(dev)
        go = dout.to(dt).contiguous()
        dd = torch.empty((r, hidden), dtype=dt, device=dev)
        dw = torch.empty((t, k), dtype=dt, device=dev)
        _native.call("qh_moe_scale_bwd", go.data_ptr(), hidden, d.data_ptr(), hidden, w.data_ptr(), inv.data_ptr(),
                     sel.data_ptr(), t, k, n_experts, hidden, dd.data_ptr(), hidden, dw.data_ptr(), code, st)
        dg = torch.empty((r, inter), dtype=dt, device=dev)
        du = torch.empty_like(dg)
        _native.call("qh_moe_down_dgrad", dd.data_ptr(), hidden, r, hidden, dn_table.data_ptr(), ldw_dn, inter,
                     seg.data_ptr(), toff.data_ptr(), n_experts, g.data_ptr(), u.data_ptr(), inter, dg.data_ptr(),
                     du.data_ptr(), inter, code, st)
        dxs = torch.empty((r, hidden), dtype=dt, device=dev)
        _native.call("qh_moe_up_dgrad", dg.data_ptr(), du.data_ptr(), inter, r, inter, gu_table.data_ptr(), ldw_gu,
                     hidden, seg.data_ptr(), toff.data_ptr(), n_experts, dxs.data_ptr(), hidden, code, st)
        dflat = torch.empty((t, hidden), dtype=dt, device=dev)
        _native.call("qh_moe_combine", dxs.data_ptr(), hidden, inv.data_ptr(), sel.data_ptr(), None, t, k, n_experts,
                     dflat.data_ptr(), hidden, code, st)
        dwg = torch.empty((n_experts, inter, hidden), dtype=dt, device=dev)
        dwu = torch.empty_like(dwg)
        dwd = torch.empty((n_experts, hidden, inter), dtype=dt, device=dev)
        _native.call("qh_moe_wgrad", 2, dg.data_ptr(), du.data_ptr(), inter, inter, xs.data_ptr(), hidden, hidden,
                     seg.data_ptr(), n_experts, dwg.data_ptr(), dwu.data_ptr(), hidden, inter * hidden, code, st)
        _native.call("qh_moe_wgrad", 1, dd.data_ptr(), None, hidden, hidden, h.data_ptr(), inter, inter,
                     seg.data_ptr(), n_experts, dwd.data_ptr(), None, inter, hidden * inter, code, st)
        wgrads = []
        for e in range(n_experts):
            wgrads.extend((dwg[e], dwu[e], dwd[e]))
        wgrads = [gr.to(dtype_) if gr.dtype != dtype_ else gr for gr, (_, dtype_) in zip(wgrads, ctx.weight_meta)]
        return (dflat, dw.to(ctx.rw_dtype), None, None, None, None, None, None, None, *wgrads)
