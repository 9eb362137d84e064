"""GPU parity of every HIP operator against the CPU oracle (same seeded inputs).

Each test also asserts that the library entry point actually ran (call counter),
so a silent fallback cannot pass.
"""
from __future__ import annotations

import pytest
import torch

from oracle import ops as O
from qwen_triton import _native
from qwen_triton import kernels as K
from qwen_triton.kernels import flash_attention as FA
from qwen_triton.kernels import matmul as MM
from qwen_triton.kernels.rope import rope_tensor

from _util import BF16_TOL, F32_TOL, close, native_calls, tol_for

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gen(seed: int) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(seed)


def randn(*shape, dtype=torch.float32, seed=0, scale=1.0):
    return (torch.randn(*shape, generator=_gen(seed)) * scale).to(dtype).to(DEV)


# ---------------------------------------------------------------------------
# elementwise
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [1, 7, 3072 * 8, 100003])
def test_residual_silu_sigmoid_forward(dtype, n):
    a, b = randn(n, dtype=dtype, seed=1), randn(n, dtype=dtype, seed=2)
    c0 = native_calls("qh_add")
    close(K.residual_add(a, b), O.residual_add(a, b), **tol_for(dtype))
    close(K.silu_mul(a, b), O.silu_mul(a, b), **tol_for(dtype))
    close(K.sigmoid_mul(a, b), O.sigmoid_mul(a, b), **tol_for(dtype))
    assert native_calls("qh_add") == c0 + 1


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gated_backward(dtype):
    g = randn(4, 513, dtype=dtype, seed=3).requires_grad_(True)
    u = randn(4, 513, dtype=dtype, seed=4).requires_grad_(True)
    go = randn(4, 513, dtype=dtype, seed=5)
    K.silu_mul(g, u).backward(go)
    eg, eu = O.silu_mul_backward(g, u, go)
    close(g.grad, eg, **tol_for(dtype))
    close(u.grad, eu, **tol_for(dtype))
    x = randn(4, 513, dtype=dtype, seed=6).requires_grad_(True)
    gt = randn(4, 513, dtype=dtype, seed=7).requires_grad_(True)
    K.sigmoid_mul(x, gt).backward(go)
    ex, eg2 = O.sigmoid_mul_backward(x, gt, go)
    close(x.grad, ex, **tol_for(dtype))
    close(gt.grad, eg2, **tol_for(dtype))


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape,dtype", [((8, 1024), torch.float32), ((64, 1024), torch.bfloat16),
                                         ((4, 5, 16, 128), torch.bfloat16), ((3, 100), torch.float32),
                                         ((2, 2048), torch.bfloat16), ((5, 16), torch.float32),
                                         ((3, 5000), torch.bfloat16)])
@pytest.mark.parametrize("one_plus", [False, True])
def test_rmsnorm_forward_backward(shape, dtype, one_plus):
    x = randn(*shape, dtype=dtype, seed=10).requires_grad_(True)
    w = randn(shape[-1], dtype=dtype, seed=11, scale=0.5).requires_grad_(True)
    go = randn(*shape, dtype=dtype, seed=12)
    y = K.rmsnorm(x, w, eps=1e-6, one_plus_weight=one_plus)
    close(y, O.rmsnorm(x, w, 1e-6, one_plus), **tol_for(dtype))
    y.backward(go)
    egx, egw = O.rmsnorm_backward(x, w, go, 1e-6, one_plus)
    close(x.grad, egx, **tol_for(dtype))
    # dW sums over all rows: compare relative to its magnitude
    tol = dict(atol=1e-3 * max(1.0, float(egw.abs().max())), rtol=1e-3) if dtype == torch.float32 else BF16_TOL
    close(w.grad, egw, **tol)


def test_rmsnorm_backward_deterministic():
    x = randn(4096, 128, dtype=torch.bfloat16, seed=13).requires_grad_(True)
    w = randn(128, dtype=torch.bfloat16, seed=14).requires_grad_(True)
    go = randn(4096, 128, dtype=torch.bfloat16, seed=15)
    grads = []
    for _ in range(2):
        x.grad = w.grad = None
        K.rmsnorm(x, w).backward(go)
        grads.append((x.grad.clone(), w.grad.clone()))
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------
def test_rope_reference_shapes_partial_rotary_fp32():
    # tests/test_kernels.py:99-107 of the reference: partial rotary 8 of 16, random cos/sin
    q, k = randn(2, 4, 5, 16, seed=20), randn(2, 4, 5, 16, seed=21)
    cos, sin = randn(2, 5, 8, seed=22), randn(2, 5, 8, seed=23)
    aq, ak = K.apply_rope(q, k, cos, sin, use_triton=True)
    close(aq, O.rope(q, cos, sin), **F32_TOL)
    close(ak, O.rope(k, cos, sin), **F32_TOL)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("backend", ["triton", "cuda_op"])
def test_rope_gqa_backward(dtype, backend):
    q = randn(2, 4, 5, 16, dtype=dtype, seed=24).requires_grad_(True)
    k = randn(2, 2, 5, 16, dtype=dtype, seed=25).requires_grad_(True)
    cos, sin = randn(2, 5, 8, dtype=dtype, seed=26), randn(2, 5, 8, dtype=dtype, seed=27)
    gq, gk = randn(2, 4, 5, 16, dtype=dtype, seed=28), randn(2, 2, 5, 16, dtype=dtype, seed=29)
    aq, ak = K.apply_rope(q, k, cos, sin, backend=backend)
    close(aq, O.rope(q, cos, sin), **tol_for(dtype))
    torch.autograd.backward((aq, ak), (gq, gk))
    close(q.grad, O.rope_backward(gq, cos, sin), **tol_for(dtype))
    close(k.grad, O.rope_backward(gk, cos, sin), **tol_for(dtype))


def test_rope_batch_broadcast_and_strided_input():
    # model layout: q comes from [B,S,H,D].transpose(1,2); cos/sin have batch 1
    B, S, H, D = 3, 7, 4, 128
    base = randn(B, S, H, D, dtype=torch.bfloat16, seed=30)
    x = base.transpose(1, 2)
    pos = torch.arange(S)
    cos, sin = O.rotary_tables(pos, D, 1e6, torch.bfloat16)
    out = rope_tensor(x, cos.to(DEV), sin.to(DEV))
    assert out.is_contiguous()
    close(out, O.rope(x, cos, sin), **BF16_TOL)


def test_rope_custom_op_registered():
    q = randn(1, 2, 3, 32, dtype=torch.bfloat16, seed=31)
    cos, sin = randn(1, 3, 32, dtype=torch.bfloat16, seed=32), randn(1, 3, 32, dtype=torch.bfloat16, seed=33)
    from qwen_triton.ops import load_rope_cuda_op

    assert load_rope_cuda_op()
    out = torch.ops.qwen_triton.rope_tensor_forward(q, cos, sin)
    close(out, O.rope(q, cos, sin), **BF16_TOL)


# ---------------------------------------------------------------------------
# KV cache
# ---------------------------------------------------------------------------
def test_write_attention_kv_known_answer():
    # tests/test_kernels.py:181-189 of the reference
    cache = torch.zeros(2, 3, 16, 8, device=DEV)
    values = randn(2, 3, 5, 8, seed=40)
    positions = torch.tensor([0, 1, 4, 7, 8], device=DEV)
    c0 = native_calls("qh_kv_write")
    out = K.write_attention_kv(cache.clone(), values, positions)
    assert native_calls("qh_kv_write") == c0 + 1
    assert torch.equal(out.cpu(), O.kv_write(cache, values, positions))


def test_write_attention_kv_strided_bf16_and_out_of_range():
    big = torch.zeros(4, 8, 64, 128, dtype=torch.bfloat16, device=DEV)
    cache = big[:, :, :32]  # strided view (capacity 64 storage)
    values = randn(4, 8, 3, 128, dtype=torch.bfloat16, seed=41)
    positions = torch.tensor([5, 31, 40], device=DEV)  # 40 is outside the view: skipped
    K.write_attention_kv(cache, values, positions)
    exp = torch.zeros(4, 8, 32, 128, dtype=torch.bfloat16)
    exp[:, :, [5, 31]] = values[:, :, :2].cpu()
    assert torch.equal(cache.cpu(), exp)
    assert torch.count_nonzero(big[:, :, 32:]).item() == 0


@pytest.mark.parametrize("S,D", [(700, 128), (64, 128), (2048, 64)])
def test_write_attention_kv_prefill_planes(S, D):
    """Prefill-sized writes (at least 1024 16-byte chunks per sequence and head: one kernel block
    row per (b, h) pair, four chunks per thread) into a strided cache view: the written rows equal
    the oracle's, positions past the view's capacity are skipped, and nothing else changes
    (S = 700 leaves a partial last block)."""
    B, H, cap = 2, 3, 2 * S
    big = torch.zeros(B, H, cap + 32, D, dtype=torch.bfloat16, device=DEV)
    cache = big[:, :, :cap]
    values = randn(B, H, S, D, dtype=torch.bfloat16, seed=44)
    positions = torch.randperm(cap + 16, generator=_gen(45))[:S]  # some land past the view: skipped
    K.write_attention_kv(cache, values, positions.to(DEV))
    keep = positions < cap
    exp = torch.zeros(B, H, cap, D, dtype=torch.bfloat16)
    exp[:, :, positions[keep]] = values.cpu()[:, :, keep]
    assert torch.equal(cache.cpu(), exp)
    assert torch.count_nonzero(big[:, :, cap:]).item() == 0


def test_append_attention_kv():
    a, b = randn(2, 3, 5, 64, dtype=torch.bfloat16, seed=42), randn(2, 3, 2, 64, dtype=torch.bfloat16, seed=43)
    assert torch.equal(K.append_attention_kv(a, b).cpu(), O.kv_append(a, b))


# ---------------------------------------------------------------------------
# Embedding
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("padding_idx", [None, 3])
def test_embedding_forward_backward(dtype, padding_idx):
    V, H = 1000, 256
    w = randn(V, H, dtype=dtype, seed=50).requires_grad_(True)
    ids = torch.randint(0, 40, (4, 33), generator=_gen(51)).to(DEV)  # many repeats
    out = K.triton_embedding(ids, w, padding_idx)
    assert torch.equal(out.cpu().float(), O.embedding(ids, w).float())
    go = randn(4, 33, H, dtype=dtype, seed=52)
    out.backward(go)
    exp = O.embedding_backward(ids, go, V, padding_idx)
    close(w.grad, exp, **tol_for(dtype))
    g1 = w.grad.clone()
    w.grad = None
    K.triton_embedding(ids, w, padding_idx).backward(go)
    assert torch.equal(g1, w.grad)


@pytest.mark.parametrize("H", [64, 20])  # row-wise vector kernel / scalar segment fallback
def test_embedding_backward_is_token_order_fp32_sum(H):
    """Each weight-gradient row is the fp32 sum of its tokens' gradient rows in token order, rounded
    once; unreferenced rows and the padding row are exactly zero."""
    V, pad = 5000, 7
    ids = torch.randint(0, 300, (3, 257), generator=_gen(53))
    ids[0, :5] = pad
    ids[2, -1] = V - 1
    go = torch.randn(3, 257, H, generator=_gen(54)).to(torch.bfloat16)
    w = torch.zeros(V, H, dtype=torch.bfloat16, device=DEV, requires_grad=True)
    K.triton_embedding(ids.to(DEV), w, pad).backward(go.to(DEV))
    exp = torch.zeros(V, H, dtype=torch.float32)
    flat_ids, flat_go = ids.reshape(-1).tolist(), go.reshape(-1, H).float()
    for t, v in enumerate(flat_ids):
        exp[v] += flat_go[t]
    exp[pad] = 0
    assert torch.equal(w.grad.cpu().view(torch.int16), exp.to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("n,wdt", [(1, torch.bfloat16), (771, torch.bfloat16), (16384, torch.bfloat16),
                                   (16385, torch.bfloat16), (4000, torch.float32)])
def test_embedding_backward_writes_every_row(n, wdt):
    """qh_embedding_bwd through the C ABI into a gradient buffer full of 7.0: every row is written
    (exact zeros for unreferenced rows and the padding row) and each hit row is the token-order
    fp32 sum rounded once (the row walk's search starts and ends its ranges at every run
    boundary whatever the token count)."""
    V, H, pad = 5000, 64, 7
    g = _gen(55)
    ids = torch.randint(0, 300, (n,), generator=g)
    ids[1:min(6, n)] = pad
    ids[-1] = V - 1
    go = torch.randn(n, H, generator=g).to(torch.bfloat16)
    gw = torch.full((V, H), 7.0, dtype=wdt, device=DEV)
    ids_d, go_d = ids.to(DEV), go.to(DEV)
    ws = _native.workspace(_native.call("qh_embedding_bwd_workspace", n, V), gw.device)
    c0 = native_calls("qh_embedding_bwd")
    _native.call("qh_embedding_bwd", ids_d.data_ptr(), go_d.data_ptr(), gw.data_ptr(), ws.data_ptr(), ws.numel(),
                 n, V, H, pad, _native.dtype_code(torch.bfloat16), _native.dtype_code(wdt), _native.stream(gw.device))
    assert native_calls("qh_embedding_bwd") == c0 + 1
    exp = torch.zeros(V, H, dtype=torch.float32)
    flat_go = go.float()
    for t, v in enumerate(ids.tolist()):
        exp[v] += flat_go[t]
    exp[pad] = 0
    exp = exp.to(wdt)
    got = gw.cpu()
    bits = torch.int16 if wdt == torch.bfloat16 else torch.int32
    assert torch.equal(got.view(bits), exp.view(bits))


def _embedding_bwd_abi(ids, go, V, pad, wdt):
    n, H = go.shape
    gw = torch.full((V, H), 7.0, dtype=wdt, device=DEV)
    ids_d, go_d = ids.to(DEV), go.to(DEV)
    ws = _native.workspace(_native.call("qh_embedding_bwd_workspace", n, V), gw.device)
    _native.call("qh_embedding_bwd", ids_d.data_ptr(), go_d.data_ptr(), gw.data_ptr(), ws.data_ptr(), ws.numel(),
                 n, V, H, pad, _native.dtype_code(go.dtype), _native.dtype_code(wdt), _native.stream(gw.device))
    return gw.cpu()


def _embedding_bwd_expected(ids, go, V, pad, wdt):
    exp = torch.zeros(V, go.shape[1], dtype=torch.float32)
    flat_go = go.float()
    for t, v in enumerate(ids.tolist()):
        if 0 <= v < V:
            exp[v] += flat_go[t]
    if 0 <= pad < V:
        exp[pad] = 0
    return exp.to(wdt)


@pytest.mark.parametrize("case", ["one_id", "one_range", "out_of_range", "tiny_vocab", "wide_rows", "f32_grad",
                                  "max_tokens", "above_max_tokens", "above_max_tokens_hot_id"])
def test_embedding_backward_id_distributions(case):
    """Every row written once, each hit row the token-order fp32 sum rounded once, for id
    distributions that load one workgroup's row range heavily (every token on one id; every token
    within a few hundred rows), ids outside [0, V) (no contribution), a vocabulary smaller than
    the workgroup count, rows wider than one 1024-column pass with a partial tail, fp32 incoming
    gradients into fp16 weights, and the token counts either side of the single-launch limit
    (32768; above it the ids are sorted first, also with one id on 30% of the tokens)."""
    g = _gen(57)
    V, H, n, pad, wdt, gdt = 5000, 64, 3000, 7, torch.bfloat16, torch.bfloat16
    if case == "one_id":
        ids = torch.full((n,), 1234, dtype=torch.int64)
    elif case == "one_range":
        n = 20000
        ids = torch.randint(4000, 4400, (n,), generator=g)
    elif case == "out_of_range":
        ids = torch.randint(-50, V + 50, (n,), generator=g)
        ids[:3] = torch.tensor([-(2 ** 40), 2 ** 40, V])
    elif case == "tiny_vocab":
        V, pad = 3, 1
        ids = torch.randint(0, V, (n,), generator=g)
    elif case == "wide_rows":
        V, H = 3000, 1032
        ids = torch.randint(0, 500, (n,), generator=g)
    elif case == "f32_grad":
        wdt, gdt = torch.float16, torch.float32
        ids = torch.randint(0, 300, (n,), generator=g)
    elif case == "max_tokens":
        V, H, n = 20000, 16, 32768
        ids = torch.randint(0, V, (n,), generator=g)
    elif case == "above_max_tokens_hot_id":  # sorted path with one run of ~12000 tokens
        V, H, n = 20000, 16, 40003
        ids = torch.randint(0, V, (n,), generator=g)
        ids[torch.rand(n, generator=g) < 0.3] = 77
    else:
        V, H, n = 20000, 16, 32769
        ids = torch.randint(0, V, (n,), generator=g)
    go = torch.randn(n, H, generator=g).to(gdt)
    got = _embedding_bwd_abi(ids, go, V, pad, wdt)
    exp = _embedding_bwd_expected(ids, go, V, pad, wdt)
    bits = torch.int16 if wdt != torch.float32 else torch.int32
    assert torch.equal(got.view(bits), exp.view(bits))


def test_embedding_backward_in_a_captured_graph():
    """qh_embedding_bwd captured in a HIP graph (the device-wide id sort and the row walk):
    every replay, with eager work between replays, equals the eager result bit for bit."""
    V, H, n, pad = 3000, 128, 2000, 3
    g = _gen(56)
    ids = torch.randint(0, 500, (n,), generator=g).to(DEV)
    go = torch.randn(n, H, generator=g).to(torch.bfloat16).to(DEV)
    ws = _native.workspace(_native.call("qh_embedding_bwd_workspace", n, V), go.device)
    gw = torch.full((V, H), 5.0, dtype=torch.bfloat16, device=DEV)

    def run():
        _native.call("qh_embedding_bwd", ids.data_ptr(), go.data_ptr(), gw.data_ptr(), ws.data_ptr(), ws.numel(),
                     n, V, H, pad, _native.dtype_code(torch.bfloat16), _native.dtype_code(torch.bfloat16),
                     _native.stream(gw.device))

    run()
    torch.cuda.synchronize()
    eager = gw.clone()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            run()
    torch.cuda.current_stream().wait_stream(s)
    for r in range(3):
        gw.fill_(float(r + 7))
        x = torch.randn(256, 256, device=DEV) @ torch.randn(256, 256, device=DEV)  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(x).all()
        assert torch.equal(gw.view(torch.int16), eager.view(torch.int16)), f"replay {r}"


# ---------------------------------------------------------------------------
# Softmax / cross-entropy
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(1000, 128), (1001, 256), (7, 5000), (3, 64)])
def test_softmax_forward_backward(shape):
    x = randn(*shape, seed=60, scale=3.0).requires_grad_(True)
    y = K.triton_softmax(x)
    close(y, O.softmax(x), **F32_TOL)
    go = randn(*shape, seed=61)
    y.backward(go)
    close(x.grad, O.softmax_backward(y, go), **F32_TOL)


@pytest.mark.parametrize("N,V,dtype", [(64, 1000, torch.float32), (8, 151936, torch.bfloat16),
                                       (5, 1001, torch.bfloat16)])
def test_cross_entropy_forward_backward(N, V, dtype):
    x = randn(N, V, dtype=dtype, seed=70, scale=2.0).requires_grad_(True)
    t = torch.randint(0, V, (N,), generator=_gen(71))
    t[1] = -100
    t = t.to(DEV)
    loss = K.triton_cross_entropy(x, t)
    eloss, _, _ = O.cross_entropy(x, t)
    close(loss, eloss, atol=1e-4, rtol=1e-4)
    loss.backward(torch.tensor(2.0, device=DEV))
    close(x.grad, O.cross_entropy_backward(x, t, 2.0), **tol_for(dtype))
    assert torch.count_nonzero(x.grad[1]).item() == 0


def test_cross_entropy_all_ignored_is_zero():
    x = randn(4, 100, seed=72)
    t = torch.full((4,), -100, device=DEV)
    assert float(K.triton_cross_entropy(x, t)) == 0.0


# ---------------------------------------------------------------------------
# MoE routing primitives
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("N,C,k", [(1000, 128, 8), (64, 4, 2), (33, 2000, 5), (16, 60, 60)])
def test_topk_bit_exact(N, C, k):
    x = randn(N, C, seed=80)
    vals, idx = K.triton_topk(x, k)
    ev, ei = O.topk(x, k)
    assert torch.equal(idx.cpu(), ei)
    assert torch.equal(vals.cpu(), ev)


@pytest.mark.parametrize("N,C,k,dtype", [(1001, 128, 8, torch.float32), (77, 128, 16, torch.bfloat16),
                                         (50, 64, 16, torch.float32), (19, 8, 8, torch.float32),
                                         (40, 16, 3, torch.float16), (16384, 128, 8, torch.float32)])
def test_topk_narrow_rows_ties_and_specials(N, C, k, dtype):
    """Rows of <= 128 columns: quantised values (many exact ties), +-0, -inf and NaN entries."""
    x = torch.round(torch.randn(N, C, generator=_gen(83)) * 2) / 2
    x[::7, 1] = -0.0
    x[::5, 2] = float("-inf")
    x[::11, 3] = float("nan")
    x[3] = float("-inf")  # a row with fewer finite values than k is still all -inf, selected by column
    x = x.to(dtype).to(DEV)
    vals, idx = K.triton_topk(x, k)
    ev, ei = O.topk(x, k)
    nan_rows = torch.isnan(x.cpu().float()).any(dim=1)
    ok = ~nan_rows
    assert torch.equal(idx.cpu()[ok], ei[ok])
    assert torch.equal(vals.cpu()[ok].view(torch.int16 if dtype != torch.float32 else torch.int32),
                       ev[ok].view(torch.int16 if dtype != torch.float32 else torch.int32))
    # NaN is never selected; rows holding one keep the order of the remaining values
    xc = x.cpu().float()
    for r in torch.nonzero(nan_rows).view(-1)[:20].tolist():
        finite = torch.where(torch.isnan(xc[r]), torch.tensor(float("-inf")), xc[r])
        order = torch.sort(-finite.double(), stable=True).indices
        order = order[~torch.isnan(xc[r][order])][:k]
        got = idx[r].cpu()
        assert torch.equal(got[:order.numel()], order)


@pytest.mark.parametrize("N,C,k,dtype", [(2, 151936, 1, torch.bfloat16), (3, 1030, 4, torch.float32),
                                         (5, 4099, 3, torch.float16)])
def test_topk_wide_rows(N, C, k, dtype):
    """Rows wider than 1024 columns (a greedy argmax over a vocabulary; widths with and without
    16-byte rows): quantised values, so the maximum is tied in several columns."""
    x = (torch.round(torch.randn(N, C, generator=_gen(84)) * 2) / 2).to(dtype).to(DEV)
    c0 = native_calls("qh_topk")
    vals, idx = K.triton_topk(x, k)
    assert native_calls("qh_topk") == c0 + 1
    ev, ei = O.topk(x, k)
    assert torch.equal(idx.cpu(), ei)
    assert torch.equal(vals.cpu(), ev)
    if k == 1:
        assert torch.equal(idx.view(-1).cpu(), torch.argmax(x.float().cpu(), dim=-1))


@pytest.mark.parametrize("N", [1, 64])
def test_topk1_wide_rows_ties_and_specials(N):
    """The greedy pick over a vocabulary row (k = 1, 151936 columns; configs 0 and 3): quantised
    values with tied maxima, +-0, -inf and NaN entries, and an all -inf row."""
    C = 151936
    x = torch.round(torch.randn(N, C, generator=_gen(85)) * 2) / 2
    x[:, ::997] = -0.0
    x[:, 5::1009] = float("-inf")
    x[::2, 11::4001] = float("nan")
    x[:, 70000] = 7.5  # a tied maximum: the lower column wins
    x[:, 150000] = 7.5
    if N > 3:
        x[3] = float("-inf")
    x = x.to(torch.bfloat16).to(DEV)
    vals, idx = K.triton_topk(x, 1)
    xc = x.cpu().float()
    ref = torch.where(torch.isnan(xc), torch.tensor(float("-inf")), xc)
    order = torch.sort(-ref.double(), dim=-1, stable=True).indices[:, 0]
    assert torch.equal(idx.view(-1).cpu(), order)
    assert torch.equal(vals.view(-1).cpu().float(), xc.gather(1, order[:, None]).view(-1))
    if N > 3:
        assert idx.view(-1)[3].item() == 0


def test_topk_ties_go_to_lowest_index():
    x = torch.tensor([[1.0, 3.0, 3.0, 0.5, 3.0, 1.0], [2.0] * 6], device=DEV)
    vals, idx = K.triton_topk(x, 4)
    assert idx.cpu().tolist() == [[1, 2, 4, 0], [0, 1, 2, 3]]
    assert torch.equal(idx.cpu(), O.topk(x, 4)[1])


def test_topk_backward_scatter():
    x = randn(10, 16, seed=81).requires_grad_(True)
    vals, idx = K.triton_topk(x, 3)
    vals.sum().backward()
    exp = torch.zeros(10, 16)
    exp.scatter_(1, idx.cpu(), 1.0)
    assert torch.equal(x.grad.cpu(), exp)


def test_one_hot_bit_exact():
    idx = torch.randint(0, 128, (100, 8), generator=_gen(82)).to(DEV)
    out = K.triton_one_hot(idx, 128)
    assert out.dtype == torch.int64 and torch.equal(out.cpu(), O.one_hot(idx, 128))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_index_add(dtype):
    tgt = randn(50, 96, dtype=dtype, seed=83)
    src = randn(300, 96, dtype=dtype, seed=84)
    index = torch.randint(0, 50, (300,), generator=_gen(85)).to(DEV)
    exp = O.index_add(tgt, src, index)
    out = K.triton_index_add(tgt.clone(), src, index)
    close(out, exp, **(F32_TOL if dtype == torch.float32 else dict(atol=5e-2, rtol=2e-2)))
    out2 = K.triton_index_add(tgt.clone(), src, index)
    assert torch.equal(out, out2)


def test_index_add_is_source_order_fp32_sum_signed_zeros():
    """fp32 index_add bit for bit against a sequential loop in source order: runs of 1 to 20 sources
    per target row (every mix of the summation's batches of four rows and single rows), targets
    holding -0.0 and +0.0, sources holding +-0.0."""
    T, D, n = 24, 40, 260
    g = _gen(90)
    tgt = torch.randn(T, D, generator=g)
    tgt[0] = -0.0
    tgt[1] = 0.0
    tgt[2, ::2] = -0.0
    src = torch.randn(n, D, generator=g)
    src[::7] = -0.0
    src[3::11] = 0.0
    counts = [1 + (r * 7) % 20 for r in range(T)]
    index = torch.cat([torch.full((c,), r) for r, c in enumerate(counts)])[:n]
    index = index[torch.randperm(index.numel(), generator=g)]
    src = src[:index.numel()]
    exp = tgt.clone()
    for j, r in enumerate(index.tolist()):
        exp[r] = exp[r] + src[j]
    out = K.triton_index_add(tgt.to(DEV), src.to(DEV), index.to(DEV))
    assert torch.equal(out.cpu().view(torch.int32), exp.view(torch.int32))


@pytest.mark.parametrize("n", [2048, 2049])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_index_add_scan_and_sorted_paths_bit_exact(n, dtype):
    """Up to 2048 source rows take the one-launch scan (each position checks whether it is the first
    of its row and adds the row's positions in order), more take the sorted path: both equal a
    sequential fp32 sum in source order, rounded once, bit for bit; indices outside [0, T) are
    skipped; one row has a run of 40 sources."""
    T, D = 300, 64
    g = _gen(91)
    tgt = torch.randn(T, D, generator=g).to(dtype)
    src = torch.randn(n, D, generator=g).to(dtype)
    index = torch.randint(-20, T + 20, (n,), generator=g)
    index[:40] = 7
    index = index[torch.randperm(n, generator=g)]
    exp = tgt.float().clone()
    for j, r in enumerate(index.tolist()):
        if 0 <= r < T:
            exp[r] = exp[r] + src[j].float()
    exp = exp.to(dtype)
    out = K.triton_index_add(tgt.to(DEV), src.to(DEV), index.to(DEV)).cpu()
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(out.view(bits), exp.view(bits))


def test_index_add_autograd():
    tgt = randn(20, 32, seed=86).requires_grad_(True)
    src = randn(40, 32, seed=87).requires_grad_(True)
    index = torch.randint(0, 20, (40,), generator=_gen(88)).to(DEV)
    out = K.triton_index_add(tgt, src, index)
    close(out, O.index_add(tgt, src, index), **F32_TOL)
    go = randn(20, 32, seed=89)
    out.backward(go)
    close(tgt.grad, go, **F32_TOL)
    close(src.grad, go[index], **F32_TOL)


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------
GEMM_SHAPES = [(1, 64, 128), (5, 300, 256), (8, 1024, 1024), (64, 1024, 1024), (200, 384, 512),
               (512, 512, 1024), (300, 520, 136), (1024, 3072, 1024), (17, 2048, 72), (33, 9000, 256),
               (40, 3072, 1024), (64, 100, 64), (16, 8200, 1000), (9, 33, 40)]


@pytest.mark.parametrize("M,N,Kd", GEMM_SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_forward(M, N, Kd, dtype):
    x = randn(M, Kd, dtype=dtype, seed=90)
    w = randn(N, Kd, dtype=dtype, seed=91, scale=0.05)
    b = randn(N, dtype=dtype, seed=92)
    c0 = native_calls("qh_gemm")
    y = K.triton_matmul(x, w, b)
    assert native_calls("qh_gemm") == c0 + 1
    close(y, O.linear(x, w, b), **BF16_TOL)


@pytest.mark.parametrize("M,N,Kd", [(64, 1024, 3072), (64, 2048, 1024), (1, 3072, 1024), (48, 1000, 1000),
                                    (9, 200, 4104), (64, 151936 // 8, 1024), (3, 20000, 136), (128, 1024, 3072),
                                    (100, 2048, 1024), (65, 6144, 1024)])
def test_gemm_decode_shapes_deterministic(M, N, Kd):
    # the small-M path splits K across 16 wavefronts and sums the slices in a fixed order
    x = randn(M, Kd, dtype=torch.bfloat16, seed=190)
    w = randn(N, Kd, dtype=torch.bfloat16, seed=191, scale=0.05)
    y0 = K.triton_matmul(x, w)
    close(y0, O.linear(x, w), **BF16_TOL)
    for _ in range(2):
        assert torch.equal(K.triton_matmul(x, w), y0)


@pytest.mark.parametrize("M", [1, 2, 5, 64, 128])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("ns", [(2048, 1024, 1000), (2048, 1024, 1024)])
def test_linear_group_matches_separate_gemms(M, with_bias, ns):
    # (2048, 1024, 1024) at M <= 4: two columns per wave in the grouped launch, one per wave in
    # the separate ones; each column is summed in the same order, so the outputs are equal. Above
    # 4 rows the chunked kernel's K slices (and so every output's summation order) depend on K
    # alone, whatever the tile shape the column count picks: equal bits at 64 and 128 rows too.
    from qwen_triton.kernels.matmul import linear_group, linear_group_ok

    Kd = 1024
    x = randn(M, Kd, dtype=torch.bfloat16, seed=200)
    ws = [randn(n, Kd, dtype=torch.bfloat16, seed=201 + i, scale=0.05) for i, n in enumerate(ns)]
    bs = [randn(w.shape[0], dtype=torch.bfloat16, seed=210 + i) if with_bias else None for i, w in enumerate(ws)]
    assert linear_group_ok(x, ws)
    c0 = native_calls("qh_gemm_multi")
    outs = linear_group(x, ws, bs)
    assert native_calls("qh_gemm_multi") == c0 + 1
    for w, b, o in zip(ws, bs, outs):
        assert torch.equal(o, K.triton_matmul(x, w, b))


@pytest.mark.parametrize("M", [1, 17, 64, 100, 128])
def test_linear_group_gated_matches_gemms_then_silu_mul(M):
    from qwen_triton.kernels.matmul import linear_group

    Kd = 1024
    x = randn(2, M, Kd, dtype=torch.bfloat16, seed=220)[0]
    wg = randn(3072, Kd, dtype=torch.bfloat16, seed=221, scale=0.05)
    wu = randn(3072, Kd, dtype=torch.bfloat16, seed=222, scale=0.05)
    fused = linear_group(x, [wg, wu], gated=True)
    assert torch.equal(fused, K.silu_mul(K.triton_matmul(x, wg), K.triton_matmul(x, wu)))
    close(fused, O.silu_mul(O.linear(x, wg), O.linear(x, wu)), atol=3e-2, rtol=3e-2)


@pytest.mark.parametrize("M", [1, 7, 20, 64, 128])
@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_linear_group_norm_prologue(M, gated, dtype):
    # rows normalised inside the launch (norm weight folded into the weights) vs rmsnorm followed
    # by the same grouped launch: the one rounding of the normalised operand is placed
    # differently, so outputs agree within a few output rounding steps; both within the band of
    # the fp64 oracle
    from qwen_triton.kernels.matmul import linear_group, linear_group_norm_ok

    Kd = 1024
    x = randn(M, Kd, dtype=dtype, seed=240, scale=3.0)
    nw = (1.0 + 0.2 * randn(Kd, dtype=torch.float32, seed=241)).to(dtype)
    # a norm weight of another dtype keeps the separate norm
    ws0 = [randn(64, Kd, dtype=dtype, seed=249, scale=0.05)]
    assert not linear_group_norm_ok(x, ws0, nw.float())
    ns = (2048, 1024, 1000) if not gated else (3072, 3072)
    ws = [randn(n, Kd, dtype=dtype, seed=242 + i, scale=0.05) for i, n in enumerate(ns)]
    assert linear_group_norm_ok(x, ws, nw, gated=gated)
    c0 = native_calls("qh_gemm_multi_rms")
    fused = linear_group(x, ws, gated=gated, norm=(nw, 1e-6, False))
    assert native_calls("qh_gemm_multi_rms") == c0 + 1
    y = K.rmsnorm(x, nw, 1e-6)
    plain = linear_group(y, ws, gated=gated)
    fused, plain = ([fused], [plain]) if gated else (fused, plain)
    # fp64 oracles with each path's rounding points: the reference rounds the normalised
    # rows (plain path); the fused path applies the row factor after the product, with the one
    # rounding on w * W (the folded weights). Both round gate and up before the SiLU-mul.
    bf = lambda t: t.to(dtype).to(torch.float64)  # noqa: E731
    xd = x.cpu().double()
    nwd = nw.cpu().double()
    inv = torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6)
    yo = bf(O.rmsnorm(x, nw, 1e-6))

    def prods(y, scale, weights):
        outs = [O.linear(y, w) * scale for w in weights]
        return [O.silu_mul(bf(outs[0]), bf(outs[1]))] if gated else outs

    r_fused_all = prods(xd, inv, [bf(w.cpu().double() * nwd[None, :]) for w in ws])
    for f, p_, r_plain, r_fused in zip(fused, plain, prods(yo, 1.0, ws), r_fused_all):
        # a few rounding steps of the largest output (one bf16 step is 2^-8 to 2^-7 relative):
        # the reference's bf16 band taken relative to the output scale
        assert (f.float() - p_.float()).abs().max().item() <= 2e-2 * p_.float().abs().max().item() + 1e-3
        close(p_, r_plain, atol=3e-2, rtol=3e-2)
        close(f, r_fused, atol=3e-2, rtol=3e-2)
    again = linear_group(x, ws, gated=gated, norm=(nw, 1e-6, False))
    for f, a in zip(fused, [again] if gated else again):
        assert torch.equal(f, a)


@pytest.mark.parametrize("M", [2, 7, 64, 128])
@pytest.mark.parametrize("gated", [False, True])
def test_gemm_multi_rms_equals_the_in_kernel_norm(M, gated):
    """qh_gemm_multi_rms on folded weights round(W * (w + 1)) vs qh_gemm_multi_ex scaling the weight
    fragments itself: bit for bit above 4 rows (the same operand rounding); at 2 rows (where
    qh_gemm_multi_ex rounds x * w instead) both within the fp64 oracle's band."""
    import ctypes

    from qwen_triton import _native

    Kd, dt = 1024, torch.bfloat16
    x = randn(M, Kd, dtype=dt, seed=290, scale=2.0)
    nw = (0.2 * randn(Kd, dtype=torch.float32, seed=291)).to(dt)
    ns = (1024, 1024) if gated else (2048, 1024, 512)
    ws = [randn(n, Kd, dtype=dt, seed=292 + i, scale=0.05) for i, n in enumerate(ns)]
    folded = [(w.float() * (nw.float() + 1.0)).to(dt) for w in ws]
    cnt = len(ws)
    outs = {}
    for name, bs in (("ex", ws), ("rms", folded)):
        o = [torch.empty(M, n, dtype=dt, device="cuda") for n in (ns[:1] if gated else ns)]
        P = ctypes.c_void_p * cnt
        L = ctypes.c_int64 * cnt
        bp, ld, nn = P(*(b.data_ptr() for b in bs)), L(*(Kd,) * cnt), L(*ns)
        cp = P(*([t.data_ptr() for t in o] + [None] * (cnt - len(o))))
        lc = L(*([t.stride(0) for t in o] + [0] * (cnt - len(o))))
        if name == "ex":
            _native.call("qh_gemm_multi_ex", M, Kd, x.data_ptr(), Kd, cnt, ctypes.addressof(bp), ctypes.addressof(ld),
                         ctypes.addressof(nn), ctypes.addressof(cp), ctypes.addressof(lc), None, None, None,
                         int(gated), nw.data_ptr(), _native.dtype_code(dt), 1e-6, 1, _native.dtype_code(dt),
                         _native.stream(x.device))
        else:
            _native.call("qh_gemm_multi_rms", M, Kd, x.data_ptr(), Kd, cnt, ctypes.addressof(bp), ctypes.addressof(ld),
                         ctypes.addressof(nn), ctypes.addressof(cp), ctypes.addressof(lc), None, int(gated), 1e-6,
                         _native.dtype_code(dt), _native.stream(x.device))
        outs[name] = o
    bf = lambda t: t.to(dt).to(torch.float64)  # noqa: E731
    xd = x.cpu().double()
    inv = torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = [O.linear(xd, f) * inv for f in folded]
    if gated:
        ref = [O.silu_mul(bf(ref[0]), bf(ref[1]))]
    for a, b, r in zip(outs["ex"], outs["rms"], ref):
        if M > 4:
            assert torch.equal(a, b)
        close(b, r, atol=3e-2, rtol=3e-2)


def test_linear_group_norm_refolds_after_an_in_place_update():
    """The folded weights are kept with the norm weight and rebuilt when a weight or the norm
    weight changes in place (version counters): results equal a fresh group on new tensors."""
    from qwen_triton.kernels.matmul import linear_group

    Kd, dt = 512, torch.bfloat16
    x = randn(16, Kd, dtype=dt, seed=300)
    nw = (1.0 + 0.1 * randn(Kd, dtype=torch.float32, seed=301)).to(dt)
    ws = [randn(256, Kd, dtype=dt, seed=302 + i, scale=0.05) for i in range(3)]
    first = linear_group(x, ws, norm=(nw, 1e-6, False))
    assert torch.equal(linear_group(x, ws, norm=(nw, 1e-6, False))[1], first[1])
    with torch.no_grad():
        ws[1].mul_(1.5)
        nw.add_(0.25)
    after = linear_group(x, ws, norm=(nw, 1e-6, False))
    fresh = linear_group(x, [w.clone() for w in ws], norm=(nw.clone(), 1e-6, False))
    for a, f, o in zip(after, fresh, first):
        assert torch.equal(a, f)
        assert not torch.equal(a, o)


def test_linear_group_norm_one_plus_and_zero_rows():
    from qwen_triton.kernels.matmul import linear_group

    Kd = 512
    x = randn(5, Kd, dtype=torch.bfloat16, seed=250)
    x[2].zero_()  # an all-zero row normalises to zero (rsqrt(eps) * 0)
    nw = 0.1 * randn(Kd, dtype=torch.bfloat16, seed=251)
    w = randn(256, Kd, dtype=torch.bfloat16, seed=252, scale=0.05)
    out = linear_group(x, [w], norm=(nw, 1e-6, True))[0]
    ref = O.linear(O.rmsnorm(x, nw, 1e-6, one_plus=True), w)
    close(out, ref, atol=3e-2, rtol=3e-2)
    assert torch.equal(out[2], torch.zeros_like(out[2]))


def test_linear_group_norm_fit_limits():
    # qh_gemm_multi_ex's in-kernel norm sums the squares of every row over all of K in both the
    # batch-1 and the chunked kernel, so every shape fits (K = 1024, 2048, 8192 at 64 rows);
    # linear_group folds the norm weight into the weights (qh_gemm_multi_rms). At K = 8192 the
    # launch without a folded copy (norm weight applied to the staged weight fragments) gives the
    # folded launch's bits.
    import ctypes

    from qwen_triton.kernels.matmul import linear_group, linear_group_norm_ok

    nn = (ctypes.c_int64 * 2)(3072, 3072)
    for kd in (1024, 2048, 8192):
        assert _native.call("qh_gemm_multi_norm_fits", 64, kd, 1, 2, ctypes.addressof(nn))
    x = randn(64, 2048, dtype=torch.bfloat16, seed=260)
    ws = [randn(3072, 2048, dtype=torch.bfloat16, seed=261 + i, scale=0.05) for i in range(2)]
    nw = (1.0 + 0.1 * randn(2048, dtype=torch.float32, seed=264)).to(torch.bfloat16)
    assert linear_group_norm_ok(x, ws, nw, gated=True)
    out = linear_group(x, ws, gated=True, norm=(nw, 1e-6, False))
    bf = lambda t: t.to(torch.bfloat16).to(torch.float64)  # noqa: E731
    xd = x.cpu().double()
    inv = torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6)
    g, u = (O.linear(xd, bf(w.cpu().double() * nw.cpu().double()[None, :])) * inv for w in ws)
    close(out, O.silu_mul(bf(g), bf(u)), atol=3e-2, rtol=3e-2)
    # K = 8192: in-kernel scaling vs folded weights, bit for bit
    kd, dt = 8192, torch.bfloat16
    x = randn(48, kd, dtype=dt, seed=265)
    nw = (0.1 * randn(kd, dtype=torch.float32, seed=266)).to(dt)
    w = randn(512, kd, dtype=dt, seed=267, scale=0.02)
    folded = (w.float() * (nw.float() + 1.0)).to(dt)
    outs = []
    for name, b in (("ex", w), ("rms", folded)):
        o = torch.empty(48, 512, dtype=dt, device="cuda")
        bp = (ctypes.c_void_p * 1)(b.data_ptr())
        ld, n1 = (ctypes.c_int64 * 1)(kd), (ctypes.c_int64 * 1)(512)
        cp, lc = (ctypes.c_void_p * 1)(o.data_ptr()), (ctypes.c_int64 * 1)(512)
        if name == "ex":
            _native.call("qh_gemm_multi_ex", 48, kd, x.data_ptr(), kd, 1, ctypes.addressof(bp), ctypes.addressof(ld),
                         ctypes.addressof(n1), ctypes.addressof(cp), ctypes.addressof(lc), None, None, None, 0,
                         nw.data_ptr(), _native.dtype_code(dt), 1e-6, 1, _native.dtype_code(dt),
                         _native.stream(x.device))
        else:
            _native.call("qh_gemm_multi_rms", 48, kd, x.data_ptr(), kd, 1, ctypes.addressof(bp), ctypes.addressof(ld),
                         ctypes.addressof(n1), ctypes.addressof(cp), ctypes.addressof(lc), None, 0, 1e-6,
                         _native.dtype_code(dt), _native.stream(x.device))
        outs.append(o)
    assert torch.equal(outs[0], outs[1])
    xd = x.cpu().double()
    inv = torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6)
    close(outs[1], O.linear(xd, folded.cpu().double()) * inv, atol=3e-2, rtol=3e-2)


@pytest.mark.parametrize("M", [1, 64, 128])
@pytest.mark.parametrize("Kd,N", [(2048, 1024), (3072, 1024), (1024, 9000)])
def test_linear_group_residual_epilogue_bitwise(M, Kd, N):
    # o_proj / down_proj with the residual add in the epilogue equal the same launch without
    # it followed by residual_add, bit for bit (and triton_matmul where it takes the decode
    # kernel, up to 8192 columns)
    from qwen_triton.kernels.matmul import linear_group

    x = randn(M, Kd, dtype=torch.bfloat16, seed=270)
    w = randn(N, Kd, dtype=torch.bfloat16, seed=271, scale=0.05)
    b = randn(N, dtype=torch.bfloat16, seed=272)
    r = randn(M, N, dtype=torch.bfloat16, seed=273, scale=4.0)
    out = linear_group(x, [w], [b], residual=[r])[0]
    assert torch.equal(out, K.residual_add(linear_group(x, [w], [b])[0], r))
    if N <= 8192:
        assert torch.equal(out, K.residual_add(K.triton_matmul(x, w, b), r))
    close(out, O.residual_add(O.linear(x, w, b).to(torch.bfloat16), r), **BF16_TOL)


def test_mlp_inference_path_matches_autograd_path():
    from qwen_triton.modules import QwenMLP

    torch.manual_seed(3)
    mlp = QwenMLP(256, 768).to(DEV, torch.bfloat16)
    x = randn(4, 3, 256, dtype=torch.bfloat16, seed=230)
    c0 = native_calls("qh_gemm_multi")
    with torch.no_grad():
        fast = mlp(x)
    assert native_calls("qh_gemm_multi") == c0 + 1
    with torch.enable_grad():
        ref = mlp(x).detach()
    assert torch.equal(fast, ref)


@pytest.mark.parametrize("M,N,Kd", [(333, 256, 192), (64, 1024, 3072), (1024, 512, 1024), (40, 96, 64)])
def test_gemm_backward_bf16(M, N, Kd):
    x = randn(2, M, Kd, dtype=torch.bfloat16, seed=93).requires_grad_(True)
    w = randn(N, Kd, dtype=torch.bfloat16, seed=94, scale=0.05).requires_grad_(True)
    b = randn(N, dtype=torch.bfloat16, seed=95).requires_grad_(True)
    go = randn(2, M, N, dtype=torch.bfloat16, seed=96)
    K.triton_matmul(x, w, b).backward(go)
    gx, gw, gb = O.linear_backward(x, w, go, need_bias=True)
    close(x.grad, gx, **BF16_TOL)
    # dW reduces over 2*M rows: scale the absolute band with sqrt(rows)
    close(w.grad, gw, atol=2e-2 * max(1.0, (2 * M) ** 0.5 / 8), rtol=2e-2)
    close(b.grad, gb, atol=2e-2 * max(1.0, (2 * M) ** 0.5 / 8), rtol=2e-2)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 1), (1, 0)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_gemm_large_tile_layouts_and_tails(ta, tb, out_dtype):
    """Shapes of >= 128 output tiles of 256x256 take the direct-to-LDS tile kernel; M, N and K all
    end in partial tiles (4000 = 15*256 + 160, 2056 = 8*256 + 8, 1000 = 15*64 + 40)."""
    M, N, Kd = 4000, 2056, 1000
    a = randn(M, Kd, dtype=torch.bfloat16, seed=300)
    b = randn(N, Kd, dtype=torch.bfloat16, seed=301, scale=0.05)
    bias = randn(N, dtype=torch.bfloat16, seed=302)
    a_op = a.t().contiguous() if ta else a  # "T" operands are stored [K, rows]
    b_op = b.t().contiguous() if tb else b
    c = torch.empty(M, N, dtype=out_dtype, device=DEV)
    _native.call("qh_gemm", ta, tb, M, N, Kd, a_op.data_ptr(), a_op.stride(0), b_op.data_ptr(), b_op.stride(0),
                 c.data_ptr(), N, bias.data_ptr(), _native.BF16, _native.dtype_code(out_dtype), _native.stream(a.device))
    ref = a.float() @ b.float().t() + bias.float()
    tol = dict(atol=2e-3, rtol=2e-3) if out_dtype == torch.float32 else BF16_TOL
    close(c, ref, **tol)
    c2 = torch.empty_like(c)
    _native.call("qh_gemm", ta, tb, M, N, Kd, a_op.data_ptr(), a_op.stride(0), b_op.data_ptr(), b_op.stride(0),
                 c2.data_ptr(), N, bias.data_ptr(), _native.BF16, _native.dtype_code(out_dtype), _native.stream(a.device))
    assert torch.equal(c, c2)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 1), (1, 0)])
@pytest.mark.parametrize("out_dtype,with_bias", [(torch.bfloat16, False), (torch.bfloat16, True),
                                                 (torch.float32, False)])
def test_gemm_persistent_tiles_with_tails(ta, tb, out_dtype, with_bias):
    """Two or more rounds of 256x256 tiles (here 33 x 17 = 561) take persistent workgroups, one per
    CU, each issuing its next tile's first k-tile load before the epilogue (16-byte rows staged in
    two halves for bf16 output without bias, register stores otherwise); M, N and K end in partial
    tiles (8229 = 32*256 + 37, 4196 = 16*256 + 100, 1000 = 15*64 + 40). Two runs are bitwise equal."""
    M, N, Kd = 8229, 4196, 1000
    a = randn(M, Kd, dtype=torch.bfloat16, seed=305)
    b = randn(N, Kd, dtype=torch.bfloat16, seed=306, scale=0.05)
    bias = randn(N, dtype=torch.bfloat16, seed=307) if with_bias else None
    a_op = a.t().contiguous() if ta else a
    b_op = b.t().contiguous() if tb else b

    def run():
        c = torch.empty(M, N, dtype=out_dtype, device=DEV)
        _native.call("qh_gemm", ta, tb, M, N, Kd, a_op.data_ptr(), a_op.stride(0), b_op.data_ptr(), b_op.stride(0),
                     c.data_ptr(), N, bias.data_ptr() if with_bias else 0, _native.BF16, _native.dtype_code(out_dtype),
                     _native.stream(a.device))
        return c

    c = run()
    ref = a.float() @ b.float().t()
    if with_bias:
        ref = ref + bias.float()
    close(c, ref, **(dict(atol=2e-3, rtol=2e-3) if out_dtype == torch.float32 else BF16_TOL))
    assert torch.equal(c, run())


@pytest.mark.parametrize("tb", [0, 1])
def test_gemm_acc_persistent_tiles(tb):
    """qh_gemm_acc (fp32 C += A B^T, the fused LM head's dX accumulation) at 33 x 17 output tiles,
    i.e. on persistent workgroups with the register epilogue at every hand-over; M and N end in
    partial tiles. Two accumulations from the same C are bitwise equal."""
    M, N, Kd = 8232, 4104, 512
    a = randn(M, Kd, dtype=torch.bfloat16, seed=320)
    b = randn(N, Kd, dtype=torch.bfloat16, seed=321, scale=0.05)
    c0 = randn(M, N, seed=322)
    b_op = b.t().contiguous() if tb else b

    def run():
        c = c0.clone()
        _native.call("qh_gemm_acc", 0, tb, M, N, Kd, a.data_ptr(), a.stride(0), b_op.data_ptr(), b_op.stride(0),
                     c.data_ptr(), N, _native.BF16, _native.stream(a.device))
        return c

    c = run()
    close(c, c0 + a.float() @ b.float().t(), atol=2e-3, rtol=2e-3)
    assert torch.equal(c, run())


@pytest.mark.parametrize("ta,tb", [(1, 1), (0, 0), (0, 1), (1, 0)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gemm_split_k(ta, tb, out_dtype):
    """Few output tiles and long K (a weight-gradient shape): K is split into fp32 partials that
    are summed in a fixed order; M and N end in partial tiles."""
    M, N, Kd = 1000, 776, 8192
    assert _native.call("qh_gemm_workspace", M, N, Kd, _native.BF16) > 0
    a = randn(M, Kd, dtype=torch.bfloat16, seed=310)
    b = randn(N, Kd, dtype=torch.bfloat16, seed=311, scale=0.05)
    bias = randn(N, dtype=torch.bfloat16, seed=312)
    a_op = a.t().contiguous() if ta else a
    b_op = b.t().contiguous() if tb else b
    c = torch.empty(M, N, dtype=out_dtype, device=DEV)
    c0 = native_calls("qh_gemm_ws")
    MM.gemm(bool(ta), bool(tb), M, N, Kd, a_op, a_op.stride(0), b_op, b_op.stride(0), c, N, bias)
    assert native_calls("qh_gemm_ws") == c0 + 1
    ref = a.float() @ b.float().t() + bias.float()
    close(c, ref, **(dict(atol=2e-3, rtol=2e-3) if out_dtype == torch.float32 else BF16_TOL))
    c2 = torch.empty_like(c)
    MM.gemm(bool(ta), bool(tb), M, N, Kd, a_op, a_op.stride(0), b_op, b_op.stride(0), c2, N, bias)
    assert torch.equal(c, c2)


def test_gemm_fp32_matches_reference_band():
    x = randn(37, 70, seed=97).requires_grad_(True)
    w = randn(45, 70, seed=98).requires_grad_(True)
    y = K.triton_matmul(x, w)
    close(y, O.linear(x, w), **F32_TOL)
    go = randn(37, 45, seed=99)
    y.backward(go)
    gx, gw, _ = O.linear_backward(x, w, go)
    close(x.grad, gx, **F32_TOL)
    close(w.grad, gw, **F32_TOL)


# ---------------------------------------------------------------------------
# Flash attention
# ---------------------------------------------------------------------------
FA_CASES = [
    # B, Hq, Hkv, Sq, Sk, D, causal, offset
    (2, 4, 2, 128, 128, 64, True, 0),
    (1, 16, 8, 300, 300, 128, True, 0),
    (2, 4, 4, 77, 77, 32, False, 0),
    (1, 2, 1, 64, 200, 128, True, 136),
    (1, 4, 1, 130, 130, 16, True, 0),
    (2, 8, 2, 1, 513, 128, False, 0),
    (1, 32, 4, 256, 256, 128, True, 0),  # GQA group 8, as config 4's attention
]


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,causal,off", FA_CASES)
def test_flash_forward(B, Hq, Hkv, Sq, Sk, D, causal, off):
    q = randn(B, Hq, Sq, D, dtype=torch.bfloat16, seed=100)
    k = randn(B, Hkv, Sk, D, dtype=torch.bfloat16, seed=101)
    v = randn(B, Hkv, Sk, D, dtype=torch.bfloat16, seed=102)
    scale = D ** -0.5
    out, lse = FA.flash_forward(q, k, v, scale, causal, Hq // Hkv, off)
    eo, el = O.attention(q, k, v, scale, causal, Hq // Hkv, off)
    close(out, eo, **BF16_TOL)
    close(lse, el, atol=2e-2, rtol=1e-3)


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,causal,off", FA_CASES + [(2, 8, 1, 100, 100, 128, True, 0),
                                                         (1, 2, 2, 70, 70, 20, True, 0)])
def test_flash_forward_fp32(B, Hq, Hkv, Sq, Sk, D, causal, off):
    """fp32 q/k/v on the fp32 matrix-core kernels (as the reference runs fp32 through its kernel):
    output and LSE against the fp64 oracle at fp32 accuracy, incl. GQA 8, a bottom-right causal
    offset, a single query and a head dim that is not a multiple of 8."""
    q = randn(B, Hq, Sq, D, seed=130)
    k = randn(B, Hkv, Sk, D, seed=131)
    v = randn(B, Hkv, Sk, D, seed=132)
    scale = D ** -0.5
    c0 = native_calls("qh_flash_fwd")
    out, lse = FA.flash_forward(q, k, v, scale, causal, Hq // Hkv, off)
    assert native_calls("qh_flash_fwd") == c0 + 1
    eo, el = O.attention(q, k, v, scale, causal, Hq // Hkv, off)
    close(out, eo, atol=2e-5, rtol=2e-5)
    close(lse, el, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal", [(1, 4, 2, 200, 128, True), (2, 2, 1, 96, 64, False),
                                                 (1, 2, 2, 130, 32, True), (1, 8, 1, 150, 128, True),
                                                 (1, 2, 1, 65, 20, False)])
def test_flash_backward_fp32(B, Hq, Hkv, S, D, causal):
    """fp32 backward (dK/dV over key blocks looping over the GQA group, dQ over query blocks) against
    the fp64 oracle's gradients; two runs bitwise equal; the public API keeps fp32 on the kernels."""
    q = randn(B, Hq, S, D, seed=140).requires_grad_(True)
    k = randn(B, Hkv, S, D, seed=141).requires_grad_(True)
    v = randn(B, Hkv, S, D, seed=142).requires_grad_(True)
    go = randn(B, Hq, S, D, seed=143)
    scale = D ** -0.5
    cf, cb = native_calls("qh_flash_fwd"), native_calls("qh_flash_bwd")
    out = K.triton_flash_attention(q, k, v, scale=scale, is_causal=causal, num_kv_groups=Hq // Hkv)
    out.backward(go)
    assert native_calls("qh_flash_fwd") == cf + 1 and native_calls("qh_flash_bwd") == cb + 1
    dq, dk, dv = O.attention_backward(q, k, v, go, scale, causal, Hq // Hkv)
    tol = dict(atol=1e-4, rtol=1e-4)
    close(q.grad, dq, **tol)
    close(k.grad, dk, **tol)
    close(v.grad, dv, **tol)
    g = (q.grad.clone(), k.grad.clone(), v.grad.clone())
    q.grad = k.grad = v.grad = None
    K.triton_flash_attention(q, k, v, scale=scale, is_causal=causal, num_kv_groups=Hq // Hkv).backward(go)
    assert torch.equal(g[0], q.grad) and torch.equal(g[1], k.grad) and torch.equal(g[2], v.grad)


def _key_valid(B, Sk, pads, holes, seed):
    kv = torch.ones(B, Sk, dtype=torch.int64)
    if pads is not None:
        for b, n in enumerate(pads):
            kv[b, :n] = 0  # left padding
    if holes:
        gen = torch.Generator().manual_seed(seed)
        kv &= (torch.rand(B, Sk, generator=gen) < 0.8).to(torch.int64)
    return kv


MASKED_CASES = [  # B, Hq, Hkv, Sq, Sk, D, left pads, random holes, window
    (3, 8, 2, 200, 200, 128, [0, 70, 150], False, 0),  # whole tiles of padding are skipped
    (2, 4, 1, 77, 300, 64, None, True, 0),  # prefill on a cache, scattered invalid keys
    (2, 4, 4, 256, 256, 128, None, False, 100),  # sliding window only
    (2, 2, 1, 130, 130, 64, [5, 64], False, 37),  # window and padding
    (4, 8, 2, 1, 333, 128, [0, 1, 100, 300], False, 0),  # padded decode step
    (1, 2, 2, 300, 300, 32, None, False, 64),  # window of exactly one tile
    (2, 4, 2, 100, 100, 64, [100, 3], False, 0),  # a sequence of padding only
    (3, 16, 2, 1, 517, 64, [0, 200, 516], True, 0),  # decode, 8 q-heads per kv-head in one block
    (2, 6, 2, 1, 90, 32, [10, 0], False, 30),  # decode, 3 q-heads per kv-head, window and padding
    (2, 4, 4, 1, 200, 128, None, False, 50),  # decode without GQA (one q-head per block)
]


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,pads,holes,window", MASKED_CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_flash_forward_masked(B, Hq, Hkv, Sq, Sk, D, pads, holes, window, dtype):
    """Padding / sliding-window masks applied in the flash kernel, against the oracle's brute force
    over the same mask (query i at cache position i + Sk - Sq); queries that see no key are zero rows
    with LSE -inf in both."""
    q = randn(B, Hq, Sq, D, dtype=dtype, seed=150)
    k = randn(B, Hkv, Sk, D, dtype=dtype, seed=151)
    v = randn(B, Hkv, Sk, D, dtype=dtype, seed=152)
    kv = _key_valid(B, Sk, pads, holes, seed=153)
    use_bits = pads is not None or holes
    bits = FA.pack_key_bits(kv.cuda()) if use_bits else None
    scale, off = D ** -0.5, Sk - Sq
    c0 = native_calls("qh_flash_fwd_masked")
    out, lse = FA.flash_forward(q, k, v, scale, True, Hq // Hkv, off, key_bits=bits, window=window)
    assert native_calls("qh_flash_fwd_masked") == c0 + 1
    eo, el = O.attention_masked(q, k, v, scale, Hq // Hkv, off, kv if use_bits else None, window or None)
    close(out, eo, **BF16_TOL)
    close(lse, el, atol=2e-2, rtol=1e-3)


def test_pack_key_bits_layout():
    """Bit j % 64 of word j // 64 is key j (bit 63 lands in the sign bit); keys past Sk are clear."""
    kv = torch.zeros(2, 130, dtype=torch.int64)
    kv[0, [0, 63, 64, 129]] = 1
    kv[1] = 1
    bits = FA.pack_key_bits(kv.cuda()).cpu()
    assert bits.shape == (2, 3)
    assert bits[0].tolist() == [1 - (1 << 63), 1, 2]
    assert bits[1].tolist() == [-1, -1, 3]


def test_flash_public_api_matches_reference_fallback_semantics():
    q = randn(1, 4, 96, 64, dtype=torch.bfloat16, seed=103)
    k = randn(1, 2, 96, 64, dtype=torch.bfloat16, seed=104)
    v = randn(1, 2, 96, 64, dtype=torch.bfloat16, seed=105)
    c0 = native_calls("qh_flash_fwd")
    out = K.triton_flash_attention(q, k, v, scale=0.125, is_causal=True, num_kv_groups=2)
    assert native_calls("qh_flash_fwd") == c0 + 1
    close(out, O.attention(q, k, v, 0.125, True, 2)[0], **BF16_TOL)


@pytest.mark.parametrize("B,Hq,Hkv,S,D,causal", [(1, 4, 2, 200, 128, True), (2, 2, 1, 96, 64, False),
                                                 (1, 2, 2, 130, 32, True), (1, 16, 2, 160, 128, True)])
def test_flash_backward(B, Hq, Hkv, S, D, causal):
    q = randn(B, Hq, S, D, dtype=torch.bfloat16, seed=110).requires_grad_(True)
    k = randn(B, Hkv, S, D, dtype=torch.bfloat16, seed=111).requires_grad_(True)
    v = randn(B, Hkv, S, D, dtype=torch.bfloat16, seed=112).requires_grad_(True)
    go = randn(B, Hq, S, D, dtype=torch.bfloat16, seed=113)
    scale = D ** -0.5
    out = K.triton_flash_attention(q, k, v, scale=scale, is_causal=causal, num_kv_groups=Hq // Hkv)
    out.backward(go)
    dq, dk, dv = O.attention_backward(q, k, v, go, scale, causal, Hq // Hkv)
    tol = dict(atol=5e-2, rtol=5e-2)
    close(q.grad, dq, **tol)
    close(k.grad, dk, **tol)
    close(v.grad, dv, **tol)
    g = (q.grad.clone(), k.grad.clone(), v.grad.clone())
    q.grad = k.grad = v.grad = None
    K.triton_flash_attention(q, k, v, scale=scale, is_causal=causal, num_kv_groups=Hq // Hkv).backward(go)
    assert torch.equal(g[0], q.grad) and torch.equal(g[1], k.grad) and torch.equal(g[2], v.grad)


@pytest.mark.parametrize("B,Hq,Hkv,Sk,D", [(3, 16, 8, 2049, 128), (1, 16, 8, 1, 128), (2, 8, 1, 100, 64),
                                           (4, 4, 4, 37, 32)])
def test_flash_decode_over_cache_slice(B, Hq, Hkv, Sk, D):
    cap = Sk + 31
    kc = randn(B, Hkv, cap, D, dtype=torch.bfloat16, seed=120)
    vc = randn(B, Hkv, cap, D, dtype=torch.bfloat16, seed=121)
    q = randn(B, Hq, 1, D, dtype=torch.bfloat16, seed=122)
    k, v = kc[:, :, :Sk], vc[:, :, :Sk]
    c0 = native_calls("qh_flash_decode")
    out = K.triton_flash_attention(q, k, v, scale=D ** -0.5, is_causal=False, num_kv_groups=Hq // Hkv)
    assert native_calls("qh_flash_decode") == c0 + 1
    close(out, O.attention(q, k, v, D ** -0.5, False, Hq // Hkv)[0], **BF16_TOL)


def test_flash_attention_unsupported_call_keeps_later_calls_on_the_kernel(monkeypatch):
    """A call the kernels do not serve (head dim 132 > 128) runs on torch for that call only; the next
    bf16 call still launches qh_flash_fwd (the flag is sticky only on a real kernel failure)."""
    import warnings

    monkeypatch.delenv("QWEN_TRITON_STRICT", raising=False)
    FA._GUARD.reset()
    q, k, v = (randn(1, 4, 64, 132, dtype=torch.bfloat16, seed=s) for s in (140, 141, 142))
    c0 = native_calls("qh_flash_fwd")
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        out = K.triton_flash_attention(q, k, v, scale=132 ** -0.5, is_causal=True, num_kv_groups=1)
    assert native_calls("qh_flash_fwd") == c0
    assert any("This call uses torch" in str(w.message) for w in rec)
    close(out, O.attention(q, k, v, 132 ** -0.5, True, 1)[0], **BF16_TOL)
    assert FA._GUARD.runtime_ok
    q, k, v = (randn(1, 4, 64, 128, dtype=torch.bfloat16, seed=s) for s in (143, 144, 145))
    out = K.triton_flash_attention(q, k, v, scale=128 ** -0.5, is_causal=True, num_kv_groups=2 // 2)
    assert native_calls("qh_flash_fwd") == c0 + 1
    close(out, O.attention(q, k, v, 128 ** -0.5, True, 1)[0], **BF16_TOL)


def test_flash_decode_device_seqlens():
    B, Hq, Hkv, cap, D = 3, 8, 4, 300, 128
    kc = randn(B, Hkv, cap, D, dtype=torch.bfloat16, seed=123)
    vc = randn(B, Hkv, cap, D, dtype=torch.bfloat16, seed=124)
    q = randn(B, Hq, 1, D, dtype=torch.bfloat16, seed=125)
    lens = [17, 300, 128]
    out = FA.flash_decode(q, kc, vc, D ** -0.5, Hq // Hkv, torch.tensor(lens, dtype=torch.int32, device=DEV))
    for b, n in enumerate(lens):
        exp = O.attention(q[b:b + 1], kc[b:b + 1, :, :n], vc[b:b + 1, :, :n], D ** -0.5, False, Hq // Hkv)[0]
        close(out[b:b + 1], exp, **BF16_TOL)


@pytest.mark.parametrize("B,Hq,Hkv,dtype", [(64, 16, 8, torch.bfloat16), (128, 32, 4, torch.bfloat16),
                                             (512, 4, 1, torch.float16), (130, 16, 4, torch.bfloat16)])
def test_flash_decode_many_sequences(B, Hq, Hkv, dtype):
    """At least 512 (sequence, kv-head) pairs with head dim 128 take the one-workgroup-per-sequence
    kernel (partials combined in LDS): per-sequence lengths including 0, 1 and non-multiples of
    the 32-key tile, GQA groups 2/8/4, checked against fp32 torch row by row; reruns bitwise equal."""
    D, cap = 128, 700
    kc = randn(B, Hkv, cap, D, dtype=dtype, seed=126)
    vc = randn(B, Hkv, cap, D, dtype=dtype, seed=127)
    q = randn(B, Hq, 1, D, dtype=dtype, seed=128)
    lens = torch.randint(0, cap + 1, (B,), generator=_gen(129))
    lens[0], lens[1], lens[2] = 0, 1, cap
    dl = lens.to(torch.int32).to(DEV)
    c0 = native_calls("qh_flash_decode")
    out = FA.flash_decode(q, kc, vc, D ** -0.5, Hq // Hkv, dl)
    assert native_calls("qh_flash_decode") == c0 + 1
    assert torch.equal(out, FA.flash_decode(q, kc, vc, D ** -0.5, Hq // Hkv, dl))
    G = Hq // Hkv
    qf = q.float().view(B, Hkv, G, D)
    s = (qf @ kc.float().transpose(-1, -2).contiguous()) * D ** -0.5  # [B, Hkv, G, cap]
    keep = torch.arange(cap, device=DEV)[None, :] < dl[:, None].long()
    s = s.masked_fill(~keep[:, None, None, :], float("-inf"))
    ref = torch.nan_to_num(torch.softmax(s, dim=-1)) @ vc.float()  # empty sequences give 0
    close(out, ref.view(B, Hq, 1, D), **BF16_TOL)
    # the full-length sequences without seqlens go through the same kernel
    full = FA.flash_decode(q, kc, vc, D ** -0.5, G)
    ref_full = torch.softmax((qf @ kc.float().transpose(-1, -2).contiguous()) * D ** -0.5, dim=-1) @ vc.float()
    close(full, ref_full.view(B, Hq, 1, D), **BF16_TOL)


@pytest.mark.parametrize("rows,cols", [(64, 1024), (3, 2048), (7, 200)])
def test_add_rmsnorm_matches_add_then_rmsnorm(rows, cols):
    from qwen_triton.kernels.rmsnorm import add_rmsnorm

    x = randn(rows, cols, dtype=torch.bfloat16, seed=240)
    r = randn(rows, cols, dtype=torch.bfloat16, seed=241)
    w = randn(cols, seed=242) * 0.1 + 1.0
    with torch.no_grad():
        s, y = add_rmsnorm(x, r, w, 1e-6, False)
        s_ref = K.residual_add(x, r)
        y_ref = K.rmsnorm(s_ref, w, eps=1e-6)
    assert torch.equal(s, s_ref) and torch.equal(y, y_ref)
    close(y, O.rmsnorm(x.double() + r.double(), w, 1e-6), atol=3e-2, rtol=3e-2)


# ---------------------------------------------------------------------------
# MoE experts: dispatch, grouped GEMM, combine
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("T,k,E", [(300, 8, 128), (64, 2, 7), (5, 1, 16)])
def test_moe_dispatch_segments_are_a_stable_sort(T, k, E):
    from qwen_triton import _native

    logits = randn(T, E, seed=250)
    sel = torch.topk(logits, k, dim=-1).indices
    w = torch.rand(T, k, generator=_gen(251)).to(DEV, torch.bfloat16)
    R = T * k
    ws = _native.workspace(_native.call("qh_moe_dispatch_workspace", T, k, E), torch.device(DEV))
    rows = torch.empty(R, dtype=torch.int32, device=DEV)
    wsorted = torch.empty(R, dtype=torch.bfloat16, device=DEV)
    inv = torch.empty(R, dtype=torch.int32, device=DEV)
    seg = torch.empty(E + 1, dtype=torch.int32, device=DEV)
    toff = torch.empty(E + 1, dtype=torch.int32, device=DEV)
    _native.call("qh_moe_dispatch", sel.data_ptr(), w.data_ptr(), T, k, E, 128, ws.data_ptr(), ws.numel(),
                 rows.data_ptr(), wsorted.data_ptr(), inv.data_ptr(), seg.data_ptr(), toff.data_ptr(), _native.BF16,
                 _native.stream(torch.device(DEV)))
    sel_c, w_c = sel.cpu().reshape(-1), w.cpu().reshape(-1)
    counts = torch.bincount(sel_c, minlength=E)
    assert torch.equal(seg.cpu().long(), torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)]))
    tiles = (counts + 127) // 128
    assert torch.equal(toff.cpu().long(), torch.cat([torch.zeros(1, dtype=torch.long), tiles.cumsum(0)]))
    order = torch.argsort(sel_c, stable=True)  # expert-major, (token, slot) order inside an expert
    assert torch.equal(rows.cpu().long(), order // k)
    assert torch.equal(wsorted.cpu(), w_c[order])
    assert torch.equal(inv.cpu().long()[order], torch.arange(R))


def _loop_experts(blk, x, w, sel):
    """The reference per-expert loop (grouped paths switched off for this call)."""
    saved = blk._grouped_ok
    blk._grouped_ok = lambda *a, **kw: False
    try:
        return blk.experts_forward(x, w, sel)
    finally:
        blk._grouped_ok = saved


def _moe_block(E, k, hidden=256, inter=128, seed=0):
    from qwen_triton import QwenTritonConfig
    from qwen_triton.modules import QwenSparseMoeBlock

    cfg = QwenTritonConfig.from_hf_config(dict(
        model_type="qwen3_moe", vocab_size=64, hidden_size=hidden, intermediate_size=512, num_hidden_layers=1,
        num_attention_heads=4, num_key_value_heads=2, head_dim=64, moe_intermediate_size=inter, num_experts=E,
        num_experts_per_tok=k, norm_topk_prob=True, decoder_sparse_step=1, mlp_only_layers=[]))
    torch.manual_seed(seed)
    blk = QwenSparseMoeBlock(cfg)
    with torch.no_grad():
        for p in blk.parameters():
            p.normal_(0.0, 0.05)
    return blk.to(DEV, torch.bfloat16)


@pytest.mark.parametrize("E,k,T", [(16, 4, 200), (32, 8, 300), (8, 1, 33)])
def test_moe_grouped_experts_match_loop(E, k, T):
    blk = _moe_block(E, k, seed=E)
    x = randn(T, 256, dtype=torch.bfloat16, seed=260)
    logits = randn(T, E, seed=261) * 2
    # route away from the last two experts: segments of zero rows
    logits[:, -2:] = -30.0
    w, sel = blk.route(logits, torch.bfloat16)
    c0 = native_calls("qh_moe_gemm")
    with torch.no_grad():
        fused = blk.experts_forward(x, w, sel)
        again = blk.experts_forward(x, w, sel)
    assert native_calls("qh_moe_gemm") == c0 + 4
    assert torch.equal(fused, again)
    loop = _loop_experts(blk, x, w, sel)
    close(fused, loop, atol=2e-2, rtol=2e-2)
    wg = torch.stack([ex.gate_proj.weight for ex in blk.experts]).float().cpu()
    wu = torch.stack([ex.up_proj.weight for ex in blk.experts]).float().cpu()
    wd = torch.stack([ex.down_proj.weight for ex in blk.experts]).float().cpu()
    ref, *_ = O.moe_block(x, None, wg, wu, wd, k, True, router_logits=logits)
    close(fused, ref, atol=3e-2, rtol=3e-2)


@pytest.mark.parametrize("E,k,T", [(4, 2, 700), (8, 2, 1100)])
def test_moe_inference_tile_path_matches_training_forward(E, k, T):
    """With many routed rows per expert the inference forward runs on the 256x256 tile kernels:
    bitwise the training forward's output, and within the bf16 band of the per-expert loop."""
    blk = _moe_block(E, k, seed=E + 200)
    x = randn(T, 256, dtype=torch.bfloat16, seed=280)
    logits = randn(T, E, seed=281) * 2
    logits[:, -1] = -30.0  # an expert without rows
    w, sel = blk.route(logits, torch.bfloat16)
    c_up, c_gemm = native_calls("qh_moe_up"), native_calls("qh_moe_gemm")
    with torch.no_grad():
        inf = blk.experts_forward(x, w, sel)
    assert native_calls("qh_moe_up") == c_up + 1 and native_calls("qh_moe_gemm") == c_gemm
    train = blk.experts_forward(x.clone().requires_grad_(True), w, sel).detach()
    assert torch.equal(inf, train)
    close(inf, _loop_experts(blk, x, w, sel), atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("E,k,T,hidden", [(4, 2, 700, 200), (8, 2, 1100, 256), (16, 4, 1200, 2048)])
def test_moe_up_gathers_token_rows(E, k, T, hidden):
    """qh_moe_up reading the token rows through the dispatch's row list (the inference forward)
    writes G, U and H bit for bit as on a gathered copy of the rows (the training forward): K tails
    (hidden not a multiple of 64), partial 256-row tiles, an expert without rows, a row stride
    past the row; H within the bf16 band of fp32 torch per expert."""
    from qwen_triton.kernels.moe_experts import TRAIN_TILE_M

    blk = _moe_block(E, k, hidden=hidden, seed=E + 300)
    ld = hidden + 24
    xfull = randn(T, ld, dtype=torch.bfloat16, seed=290)
    logits = randn(T, E, seed=291) * 2
    logits[:, -1] = -30.0  # an expert without rows
    w, sel = blk.route(logits, torch.bfloat16)
    sel, w = sel.contiguous(), w.contiguous()
    r, inter, bf = T * k, 128, torch.bfloat16
    code, st = _native.dtype_code(bf), _native.stream(xfull.device)
    ws = _native.workspace(_native.call("qh_moe_dispatch_workspace", T, k, E), xfull.device)
    rows = torch.empty(r, dtype=torch.int32, device=DEV)
    wsorted = torch.empty(r, dtype=bf, device=DEV)
    inv = torch.empty(r, dtype=torch.int32, device=DEV)
    seg = torch.empty(E + 1, dtype=torch.int32, device=DEV)
    toff = torch.empty_like(seg)
    _native.call("qh_moe_dispatch", sel.data_ptr(), w.data_ptr(), T, k, E, TRAIN_TILE_M, ws.data_ptr(), ws.numel(),
                 rows.data_ptr(), wsorted.data_ptr(), inv.data_ptr(), seg.data_ptr(), toff.data_ptr(), code, st)
    xs = torch.empty(r, hidden, dtype=bf, device=DEV)
    _native.call("qh_moe_gather", xfull.data_ptr(), ld, rows.data_ptr(), r, hidden, xs.data_ptr(), hidden, code, st)
    gu, _ = blk._expert_tables(xfull.device)
    ldw = blk.experts[0].gate_proj.weight.stride(0)

    def up(a, lda, row_list):
        g, u, h = (torch.full((r, inter), 7.0, dtype=bf, device=DEV) for _ in range(3))
        _native.call("qh_moe_up", a.data_ptr(), lda, row_list, r, hidden, gu.data_ptr(), ldw, inter, seg.data_ptr(),
                     toff.data_ptr(), E, g.data_ptr(), u.data_ptr(), h.data_ptr(), inter, code, st)
        return g, u, h

    ref = up(xs, hidden, None)
    got = up(xfull, ld, rows.data_ptr())
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    segs = seg.cpu().tolist()
    assert segs[E] - segs[E - 1] == 0 and max(b - a for a, b in zip(segs, segs[1:])) > TRAIN_TILE_M
    xr = xfull[:, :hidden][rows.long()].float()
    for e in range(E):
        a, b = segs[e], segs[e + 1]
        if a == b:
            continue
        gref = xr[a:b] @ blk.experts[e].gate_proj.weight.float().t()
        uref = xr[a:b] @ blk.experts[e].up_proj.weight.float().t()
        close(got[2][a:b].float(), torch.nn.functional.silu(gref) * uref, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("E,k,T", [(8, 2, 300), (4, 2, 700), (16, 4, 257)])
def test_moe_grouped_training_matches_loop_gradients(E, k, T):
    """Autograd through the grouped training kernels vs the per-expert loop: output and the
    gradients of the input, the router logits and every expert weight (segments of 0, < 256 and
    > 256 rows)."""
    blk = _moe_block(E, k, seed=E + 100)
    x0 = randn(T, 256, dtype=torch.bfloat16, seed=270)
    l0 = randn(T, E, seed=271) * 2
    l0[:, -1] = -30.0  # an expert without rows
    go = randn(T, 256, dtype=torch.bfloat16, seed=272)

    def run(grouped):
        x = x0.clone().requires_grad_(True)
        logits = l0.clone().requires_grad_(True)
        for p in blk.parameters():
            p.grad = None
        w, sel = blk.route(logits, torch.bfloat16)
        out = blk.experts_forward(x, w, sel) if grouped else _loop_experts(blk, x, w, sel)
        out.backward(go)
        wg = [torch.zeros_like(p) if p.grad is None else p.grad.clone()
              for e in blk.experts for p in (e.gate_proj.weight, e.up_proj.weight, e.down_proj.weight)]
        return out.detach(), x.grad.clone(), logits.grad.clone(), wg

    c_up, c_wg = native_calls("qh_moe_up"), native_calls("qh_moe_wgrad")
    out, gx, gl, gw = run(True)
    assert native_calls("qh_moe_up") == c_up + 1 and native_calls("qh_moe_wgrad") == c_wg + 2
    out2, gx2, gl2, gw2 = run(True)
    assert torch.equal(out, out2) and torch.equal(gx, gx2) and torch.equal(gl, gl2)
    assert all(torch.equal(a, b) for a, b in zip(gw, gw2))
    rout, rgx, rgl, rgw = run(False)
    close(out, rout, atol=2e-2, rtol=2e-2)
    close(gx, rgx, atol=2e-2, rtol=2e-2)
    close(gl, rgl, atol=2e-2, rtol=2e-2)
    for a, b in zip(gw, rgw):
        scale = max(1.0, float(b.abs().max()))
        close(a, b, atol=2e-2 * scale, rtol=2e-2)
    # the expert without rows has exactly zero weight gradients
    assert all(int(torch.count_nonzero(t)) == 0 for t in gw[-3:])


def _decode_step_inputs(B, Hq, Hkv, D, cap, seed):
    q2 = randn(B, Hq * D, dtype=torch.bfloat16, seed=seed)
    k2 = randn(B, Hkv * D, dtype=torch.bfloat16, seed=seed + 1, scale=2.0)
    v2 = randn(B, Hkv * D, dtype=torch.bfloat16, seed=seed + 2)
    kc = randn(B, Hkv, cap, D, dtype=torch.bfloat16, seed=seed + 3)
    vc = randn(B, Hkv, cap, D, dtype=torch.bfloat16, seed=seed + 4)
    qw = (1.0 + 0.2 * randn(D, seed=seed + 5)).to(torch.bfloat16)
    kw = (1.0 + 0.2 * randn(D, seed=seed + 6)).to(torch.bfloat16)
    return q2, k2, v2, kc, vc, qw, kw


@pytest.mark.parametrize("Hq,Hkv,B", [(16, 8, 64), (32, 8, 64), (8, 8, 70)])
@pytest.mark.parametrize("p", [0, 1, 15, 16, 31, 32, 200, 383, 500, 639])
@pytest.mark.parametrize("cdtype", [torch.bfloat16])
def test_flash_decode_prepare_matches_prepare_then_decode(Hq, Hkv, B, p, cdtype):
    # the decode step that prepares its own rows equals the prepare pass followed by the decode
    # kernel bit for bit: output and the whole caches (new rows at p, nothing else touched).
    # p < 384 puts the new row in its wave's first three key tiles (written, then drained, before
    # that tile is read); larger p relies on the loop's own wait before the third tile
    D, cap = 128, 640
    assert _native.call("qh_flash_decode_prepare_ok", B, Hq, Hkv, p + 1, D) == 1
    q2, k2, v2, kc, vc, qw, kw = _decode_step_inputs(B, Hq, Hkv, D, cap, seed=300 + p)
    theta = (p * torch.pow(1e6, -torch.arange(0, D, 2, dtype=torch.float64) / D)).float()
    cos = torch.cat([theta.cos(), theta.cos()]).view(1, 1, D).to(cdtype).to(DEV)
    sin = torch.cat([theta.sin(), theta.sin()]).view(1, 1, D).to(cdtype).to(DEV)
    pos = torch.tensor([p], dtype=torch.long, device=DEV)
    sk = p + 1
    code = _native.dtype_code
    st = _native.stream(torch.device(DEV))
    # reference: prepare pass, then the decode kernel over keys [0, sk)
    kc_r, vc_r = kc.clone(), vc.clone()
    q_r = torch.empty((B, Hq, 1, D), dtype=torch.bfloat16, device=DEV)
    _native.call("qh_attn_prepare", q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0), v2.data_ptr(),
                 v2.stride(0), qw.data_ptr(), kw.data_ptr(), 1e-6, 0, cos.data_ptr(), sin.data_ptr(), cos.stride(0),
                 cos.stride(1), 1, D, q_r.data_ptr(), kc_r.data_ptr(), *kc_r.stride()[:3], vc_r.data_ptr(),
                 *vc_r.stride()[:3], pos.data_ptr(), B, 1, Hq, Hkv, D, cap, code(torch.bfloat16), code(qw.dtype),
                 code(cdtype), st)
    o_r = FA.flash_decode(q_r, kc_r[:, :, :sk], vc_r[:, :, :sk], D ** -0.5, Hq // Hkv)
    # fused
    o = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=DEV)
    c0 = native_calls("qh_flash_decode_prepare")
    _native.call("qh_flash_decode_prepare", q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0), v2.data_ptr(),
                 v2.stride(0), qw.data_ptr(), kw.data_ptr(), 1e-6, 0, cos.data_ptr(), sin.data_ptr(), cos.stride(0),
                 1, D, kc.data_ptr(), *kc.stride()[:3], vc.data_ptr(), *vc.stride()[:3], cap, pos.data_ptr(),
                 o.data_ptr(), None, None, B, Hq, Hkv, sk, D, D ** -0.5, code(torch.bfloat16), code(qw.dtype),
                 code(cdtype), st)
    assert native_calls("qh_flash_decode_prepare") == c0 + 1
    assert torch.equal(kc, kc_r) and torch.equal(vc, vc_r)
    assert torch.equal(o, o_r.view(B, Hq, D))
    # and against the oracle: attention over the prepared rows
    qo = q_r.view(B, Hq, 1, D)
    close(o.view(B, Hq, 1, D), O.attention(qo, kc_r[:, :, :sk], vc_r[:, :, :sk], D ** -0.5, False, Hq // Hkv)[0],
          **BF16_TOL)


def test_flash_decode_prepare_rejects_fp32_cos():
    # fp32 cos/sin would make the rotation's products inexact, and the fused rows could then differ
    # from the prepare pass's by the compiler's multiply-add contraction: the entry point refuses
    B, Hq, Hkv, D, cap = 64, 16, 8, 128, 64
    q2, k2, v2, kc, vc, qw, kw = _decode_step_inputs(B, Hq, Hkv, D, cap, seed=340)
    cos = torch.rand(1, 1, D, device=DEV)
    pos = torch.tensor([3], dtype=torch.long, device=DEV)
    o = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=DEV)
    code = _native.dtype_code
    with pytest.raises(_native.NativeError, match="activation dtype"):
        _native.call("qh_flash_decode_prepare", q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0),
                     v2.data_ptr(), v2.stride(0), qw.data_ptr(), kw.data_ptr(), 1e-6, 0, cos.data_ptr(),
                     cos.data_ptr(), cos.stride(0), 1, D, kc.data_ptr(), *kc.stride()[:3], vc.data_ptr(),
                     *vc.stride()[:3], cap, pos.data_ptr(), o.data_ptr(), None, None, B, Hq, Hkv, 4, D, D ** -0.5,
                     code(torch.bfloat16), code(qw.dtype), code(torch.float32), _native.stream(torch.device(DEV)))


def test_flash_decode_prepare_static_cache_seqlens():
    # captured-step form: keys span the whole cache, each sequence's valid length from seqlens
    B, Hq, Hkv, D, cap, p = 64, 16, 8, 128, 160, 100
    q2, k2, v2, kc, vc, qw, kw = _decode_step_inputs(B, Hq, Hkv, D, cap, seed=330)
    cos = torch.rand(1, 1, D, device=DEV).to(torch.bfloat16)
    sin = torch.rand(1, 1, D, device=DEV).to(torch.bfloat16)
    pos = torch.tensor([p], dtype=torch.long, device=DEV)
    seqlens = torch.randint(p + 1, cap + 1, (B,), generator=_gen(331), dtype=torch.int32).to(DEV)
    code = _native.dtype_code
    st = _native.stream(torch.device(DEV))
    kc_r, vc_r = kc.clone(), vc.clone()
    q_r = torch.empty((B, Hq, 1, D), dtype=torch.bfloat16, device=DEV)
    _native.call("qh_attn_prepare", q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0), v2.data_ptr(),
                 v2.stride(0), qw.data_ptr(), kw.data_ptr(), 1e-6, 1, cos.data_ptr(), sin.data_ptr(), cos.stride(0),
                 cos.stride(1), 1, D, q_r.data_ptr(), kc_r.data_ptr(), *kc_r.stride()[:3], vc_r.data_ptr(),
                 *vc_r.stride()[:3], pos.data_ptr(), B, 1, Hq, Hkv, D, cap, code(torch.bfloat16), code(qw.dtype),
                 code(torch.bfloat16), st)
    o_r = FA.flash_decode(q_r, kc_r, vc_r, D ** -0.5, Hq // Hkv, seqlens=seqlens)
    o = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=DEV)
    _native.call("qh_flash_decode_prepare", q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0), v2.data_ptr(),
                 v2.stride(0), qw.data_ptr(), kw.data_ptr(), 1e-6, 1, cos.data_ptr(), sin.data_ptr(), cos.stride(0),
                 1, D, kc.data_ptr(), *kc.stride()[:3], vc.data_ptr(), *vc.stride()[:3], cap, pos.data_ptr(),
                 o.data_ptr(), None, seqlens.data_ptr(), B, Hq, Hkv, cap, D, D ** -0.5, code(torch.bfloat16),
                 code(qw.dtype), code(torch.bfloat16), st)
    assert torch.equal(kc, kc_r) and torch.equal(vc, vc_r)
    assert torch.equal(o, o_r.view(B, Hq, D))


@pytest.mark.parametrize("B", [1, 3])
@pytest.mark.parametrize("p", [0, 37, 200, 511])
def test_flash_decode_prepare_short_context_small_batch(B, p):
    # few sequences with at most 512 keys also take the workgroup kernel that prepares its own rows
    # (the split kernel otherwise serves them, summing in another order): cache rows bitwise equal
    # to the prepare pass, output within the bf16 band of the fp64 oracle over the prepared rows
    Hq, Hkv, D, cap = 16, 8, 128, 640
    sk = p + 1
    assert _native.call("qh_flash_decode_prepare_ok", B, Hq, Hkv, sk, D) == 1
    assert _native.call("qh_flash_decode_prepare_ok", B, Hq, Hkv, 513, D) == 0
    q2, k2, v2, kc, vc, qw, kw = _decode_step_inputs(B, Hq, Hkv, D, cap, seed=360 + p)
    theta = (p * torch.pow(1e6, -torch.arange(0, D, 2, dtype=torch.float64) / D)).float()
    cos = torch.cat([theta.cos(), theta.cos()]).view(1, 1, D).to(torch.bfloat16).to(DEV)
    sin = torch.cat([theta.sin(), theta.sin()]).view(1, 1, D).to(torch.bfloat16).to(DEV)
    pos = torch.tensor([p], dtype=torch.long, device=DEV)
    code = _native.dtype_code
    st = _native.stream(torch.device(DEV))
    kc_r, vc_r = kc.clone(), vc.clone()
    q_r = torch.empty((B, Hq, 1, D), dtype=torch.bfloat16, device=DEV)
    _native.call("qh_attn_prepare", q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0), v2.data_ptr(),
                 v2.stride(0), qw.data_ptr(), kw.data_ptr(), 1e-6, 0, cos.data_ptr(), sin.data_ptr(), cos.stride(0),
                 cos.stride(1), 1, D, q_r.data_ptr(), kc_r.data_ptr(), *kc_r.stride()[:3], vc_r.data_ptr(),
                 *vc_r.stride()[:3], pos.data_ptr(), B, 1, Hq, Hkv, D, cap, code(torch.bfloat16), code(qw.dtype),
                 code(torch.bfloat16), st)
    o = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=DEV)
    for _ in range(2):  # reruns are bitwise equal
        _native.call("qh_flash_decode_prepare", q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0),
                     v2.data_ptr(), v2.stride(0), qw.data_ptr(), kw.data_ptr(), 1e-6, 0, cos.data_ptr(),
                     sin.data_ptr(), cos.stride(0), 1, D, kc.data_ptr(), *kc.stride()[:3], vc.data_ptr(),
                     *vc.stride()[:3], cap, pos.data_ptr(), o.data_ptr(), None, None, B, Hq, Hkv, sk, D, D ** -0.5,
                     code(torch.bfloat16), code(qw.dtype), code(torch.bfloat16), st)
        o0 = o.clone() if _ == 0 else o0
    assert torch.equal(o, o0)
    assert torch.equal(kc, kc_r) and torch.equal(vc, vc_r)
    ref = O.attention(q_r, kc_r[:, :, :sk], vc_r[:, :, :sk], D ** -0.5, False, Hq // Hkv)[0]
    close(o.view(B, Hq, 1, D), ref, **BF16_TOL)
    o_split = FA.flash_decode(q_r, kc_r[:, :, :sk], vc_r[:, :, :sk], D ** -0.5, Hq // Hkv)
    close(o.view(B, Hq, 1, D), o_split, atol=1e-2, rtol=1e-2)


# ---------------------------------------------------------------------------
# fused LM head + cross-entropy
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("N,H,V,chunk", [(300, 64, 1000, 128), (517, 128, 4096, 256), (64, 256, 392, 8192),
                                         (700, 64, 2056, 300)])
def test_fused_linear_cross_entropy_matches_unfused_and_oracle(N, H, V, chunk, monkeypatch):
    """Loss, dX and dW of the fused op against (a) the unfused HIP path (triton_matmul + triton_cross_entropy,
    same bf16 rounding of the logits: equal up to fp32 summation order) and (b) fp64 autograd of the
    oracle's linear + cross-entropy (bf16 band). Targets include ignored rows; vocab sizes are not tile
    multiples; several row blocks (`chunk` rows each), the last one partial."""
    from qwen_triton.kernels import linear_cross_entropy as LCE

    monkeypatch.setattr(LCE, "ROW_CHUNK", chunk)
    x0 = randn(N, H, dtype=torch.bfloat16, seed=150)
    w0 = randn(V, H, dtype=torch.bfloat16, seed=151, scale=0.1)
    t = torch.randint(0, V, (N,), generator=_gen(152))
    t[::7] = -100
    t = t.to(DEV)
    x, w = x0.clone().requires_grad_(True), w0.clone().requires_grad_(True)
    c0 = native_calls("qh_lmce_rows_fwd")
    loss = K.fused_linear_cross_entropy(x, w, t)
    loss.backward()
    assert native_calls("qh_lmce_rows_fwd") == c0 + (N + chunk - 1) // chunk
    xu, wu = x0.clone().requires_grad_(True), w0.clone().requires_grad_(True)
    lu = K.triton_cross_entropy(K.triton_matmul(xu, wu), t)
    lu.backward()
    assert abs(float(loss) - float(lu)) <= 1e-5 * abs(float(lu))
    close(x.grad, xu.grad, atol=2e-3 * float(xu.grad.abs().max()), rtol=1e-2)
    close(w.grad, wu.grad, atol=2e-3 * float(wu.grad.abs().max()), rtol=1e-2)
    # fp64 oracle autograd
    xd = x0.double().cpu().requires_grad_(True)
    wd = w0.double().cpu().requires_grad_(True)
    lo = torch.nn.functional.cross_entropy(xd @ wd.T, t.cpu(), ignore_index=-100)
    lo.backward()
    assert abs(float(loss) - float(lo)) <= 2e-2 * abs(float(lo))
    close(x.grad, xd.grad, atol=3e-2 * float(xd.grad.abs().max()), rtol=3e-2)
    close(w.grad, wd.grad, atol=3e-2 * float(wd.grad.abs().max()), rtol=3e-2)
    # forward without autograd (no logits at all, 256-column partials) gives the same loss up to the
    # fp32 order of the partial merge; the upstream gradient scales the gradients; reruns are bitwise equal
    c1 = native_calls("qh_lmce_fwd")
    with torch.no_grad():
        l0 = K.fused_linear_cross_entropy(x0, w0, t)
    assert native_calls("qh_lmce_fwd") == c1 + 1
    assert abs(float(l0) - float(loss)) <= 1e-6 * abs(float(loss))
    x3, w3 = x0.clone().requires_grad_(True), w0.clone().requires_grad_(True)
    (K.fused_linear_cross_entropy(x3, w3, t) * 0.5).backward()
    close(x3.grad, x.grad.float() * 0.5, atol=1e-3 * float(x.grad.abs().max()), rtol=1e-2)
    close(w3.grad, w.grad.float() * 0.5, atol=1e-3 * float(w.grad.abs().max()), rtol=1e-2)
    x2, w2 = x0.clone().requires_grad_(True), w0.clone().requires_grad_(True)
    K.fused_linear_cross_entropy(x2, w2, t).backward()
    assert torch.equal(x2.grad, x.grad) and torch.equal(w2.grad, w.grad)


def test_fused_linear_cross_entropy_all_rows_ignored():
    x = randn(40, 64, dtype=torch.bfloat16, seed=153).requires_grad_(True)
    w = randn(256, 64, dtype=torch.bfloat16, seed=154).requires_grad_(True)
    t = torch.full((40,), -100, device=DEV)
    loss = K.fused_linear_cross_entropy(x, w, t)
    loss.backward()
    assert float(loss) == 0.0
    assert float(x.grad.abs().max()) == 0.0 and float(w.grad.abs().max()) == 0.0


# ---------------------------------------------------------------------------
# gated delta rule (Qwen3-Next linear attention)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B,S,H,K,V,dtype,init", [
    (2, 37, 3, 16, 8, torch.float32, False), (2, 37, 3, 16, 8, torch.float32, True),
    (1, 300, 4, 128, 128, torch.bfloat16, True), (3, 65, 2, 64, 100, torch.bfloat16, False),
    (1, 1, 8, 128, 128, torch.float16, True), (2, 0, 2, 32, 32, torch.bfloat16, True)])
def test_gated_delta_rule_matches_oracle(B, S, H, K, V, dtype, init):
    """One launch over the whole sequence against the fp64 recurrence: outputs, final state, an initial
    state, value widths that are not multiples of the 64-column block, a single token and an empty
    sequence (the state passes through)."""
    from qwen_triton.kernels import gated_delta_rule_sequence

    q = randn(B, S, H, K, seed=160)
    k = randn(B, S, H, K, seed=161)
    q, k = (q / q.norm(dim=-1, keepdim=True)).to(dtype), (k / k.norm(dim=-1, keepdim=True)).to(dtype)
    v = randn(B, S, H, V, dtype=dtype, seed=162)
    g = -randn(B, S, H, seed=163).abs() * 0.2
    beta = torch.sigmoid(randn(B, S, H, seed=164))
    s0 = randn(B, H, K, V, seed=165, scale=0.5) if init else None
    c0 = native_calls("qh_gated_delta_rule")
    out, st = gated_delta_rule_sequence(q, k, v, g, beta, initial_state=s0)
    assert native_calls("qh_gated_delta_rule") == c0 + 1
    assert out.dtype == dtype and st.dtype == torch.float32 and st.shape == (B, H, K, V)
    eo, es = O.gated_delta_rule(q, k, v, g, beta, s0)
    tol = F32_TOL if dtype == torch.float32 else BF16_TOL
    close(out, eo, **tol)
    close(st, es, atol=1e-3 if dtype == torch.float32 else 3e-2, rtol=1e-3 if dtype == torch.float32 else 3e-2)
    # chunked in two launches through the state = one launch
    if S >= 2:
        h = S // 2
        o1, s1 = gated_delta_rule_sequence(q[:, :h], k[:, :h], v[:, :h], g[:, :h], beta[:, :h], initial_state=s0)
        o2, s2 = gated_delta_rule_sequence(q[:, h:], k[:, h:], v[:, h:], g[:, h:], beta[:, h:], initial_state=s1)
        assert torch.equal(torch.cat((o1, o2), dim=1), out) and torch.equal(s2, st)


# ---------------------------------------------------------------------------
# greedy decode step
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B,V", [(1, 151936), (3, 1000), (64, 4104), (64, 151936), (2, 8)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_greedy_step_is_argmax_and_advances_the_state(B, V, dtype):
    """qh_greedy_step against torch.argmax of the same values (ties to the lowest column, NaN the
    largest), the token written at the device column, the counters advanced; a column past the
    buffer stores nothing."""
    x = randn(B, V, dtype=dtype, seed=300)
    if V >= 8:
        top = x.float().max(dim=-1).values
        x[0, V // 2] = top[0].to(dtype)          # tie with the row's maximum at a later column
        x[0, 1] = top[0].to(dtype)               # and an earlier one: the earliest wins
    if B >= 3:
        x[2, V - 1] = float("nan")               # NaN is the largest value
        x[2, V - 3] = float("nan")
    if B >= 2 and V >= 8:
        x[1] = -x[1].abs() - 1                   # a row whose maximum is zero, -0.0 before +0.0:
        x[1, 3] = -0.0                           # they compare equal, the earlier column wins
        x[1, 7] = 0.0
    expect = x.float().cpu().argmax(dim=-1)
    if B >= 2 and V >= 8:
        assert int(expect[1]) == 3
    ids = torch.full((B, 1), -5, dtype=torch.long, device=DEV)
    tokens = torch.full((B, 6), -7, dtype=torch.long, device=DEV)
    col = torch.full((1, 1), 2, dtype=torch.long, device=DEV)
    pos = torch.full((1,), 40, dtype=torch.long, device=DEV)
    lens = torch.arange(B, dtype=torch.int32, device=DEV) + 10
    ws = _native.workspace(_native.call("qh_greedy_step_workspace", B, V), x.device)
    c0 = native_calls("qh_greedy_step")

    def step():
        _native.call("qh_greedy_step", x.data_ptr(), x.stride(0), B, V, ids.data_ptr(), tokens.data_ptr(),
                     tokens.stride(0), tokens.shape[1], col.data_ptr(), pos.data_ptr(), lens.data_ptr(),
                     ws.data_ptr(), ws.numel(), _native.dtype_code(dtype), _native.stream(x.device))

    step()
    assert native_calls("qh_greedy_step") == c0 + 1
    assert torch.equal(ids[:, 0].cpu(), expect)
    assert torch.equal(tokens[:, 2].cpu(), expect)
    assert (tokens[:, [0, 1, 3, 4, 5]] == -7).all()
    assert int(col) == 3 and int(pos) == 41
    assert torch.equal(lens.cpu(), torch.arange(B, dtype=torch.int32) + 11)
    col.fill_(6)  # past the token buffer: ids still written, no token stored
    ids.fill_(-5)
    step()
    assert torch.equal(ids[:, 0].cpu(), expect) and (tokens[:, [0, 1, 3, 4, 5]] == -7).all()
    assert int(col) == 7 and int(pos) == 42
