"""Expert computation of the sparse MoE block as dispatch + grouped GEMM + combine.

Reference: the per-expert loop of ``QwenSparseMoeBlock.forward``
(qwen_triton/modules/moe.py:45-51): one-hot/nonzero/where to find each
expert's tokens, the expert SwiGLU MLP on them, scaling by the routing weight
and ``triton_index_add`` into a zero tensor in ascending expert order.

Here the routed (token, slot) pairs are sorted by expert once
(``qh_moe_dispatch``), both expert GEMMs run as one grouped launch each over
all experts (``qh_moe_gemm``: gate/up with the token gather and SiLU-mul fused,
down with the routing-weight scaling fused), and ``qh_moe_combine`` sums each
token's expert rows in ascending expert order with the reference's bf16
rounding after every add. No host synchronisation; deterministic.
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
    _native.call("qh_moe_combine", y.data_ptr(), hidden, inv.data_ptr(), sel.data_ptr(), t, k, n_experts,
                 out.data_ptr(), hidden, code, st)
    return out
