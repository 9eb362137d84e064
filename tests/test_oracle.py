"""Pins the CPU oracle against independent authorities (CPU only).

Each oracle function is checked against something that does not restate its
formula: torch built-ins (SDPA, cross_entropy, softmax, topk, index_add_,
one_hot, embedding, linear), autograd of the forward, HF transformers' Qwen3 /
Qwen3-MoE code (the reference's ``ref`` backend), complex-number rotation,
adjoint identities, brute-force loops, and the reference's own known-answer
test. A plausible slip (dropped term, wrong sign, transposed operand, wrong
tie rule) fails at least one of them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops as O

D64 = torch.float64


def g(seed):
    return torch.Generator().manual_seed(seed)


def rn(*shape, seed=0, dtype=D64):
    return torch.randn(*shape, generator=g(seed), dtype=dtype)


# ---------------------------------------------------------------- attention
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("groups", [1, 2, 4])
def test_attention_matches_sdpa_and_lse(causal, groups):
    q = rn(2, 4, 9, 16, seed=1)
    k = rn(2, 4 // groups, 9, 16, seed=2)
    v = rn(2, 4 // groups, 9, 16, seed=3)
    out, lse = O.attention(q, k, v, 0.25, causal, groups)
    ke, ve = k.repeat_interleave(groups, 1), v.repeat_interleave(groups, 1)
    ref = F.scaled_dot_product_attention(q, ke, ve, is_causal=causal, scale=0.25)
    torch.testing.assert_close(out, ref)
    s = (q @ ke.transpose(-1, -2)) * 0.25
    if causal:
        s = s.masked_fill(torch.ones(9, 9, dtype=torch.bool).triu(1), float("-inf"))
    torch.testing.assert_close(lse, torch.logsumexp(s, -1))


def test_attention_bottom_right_offset_equals_explicit_mask():
    q, k, v = rn(1, 2, 3, 8, seed=4), rn(1, 2, 7, 8, seed=5), rn(1, 2, 7, 8, seed=6)
    out, _ = O.attention(q, k, v, 0.3, True, 1, causal_offset=4)
    mask = torch.tensor([[j <= i + 4 for j in range(7)] for i in range(3)])
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=0.3)
    torch.testing.assert_close(out, ref)


def test_masked_attention_reduces_to_causal_without_padding_or_window():
    q, k, v = rn(2, 4, 5, 8, seed=7), rn(2, 2, 9, 8, seed=8), rn(2, 2, 9, 8, seed=9)
    exp = O.attention(q, k, v, 0.4, True, 2, causal_offset=4)
    for kv, win in ((None, None), (torch.ones(2, 9), None), (None, 14)):  # a window of 14 covers every key
        got = O.attention_masked(q, k, v, 0.4, 2, 4, kv, win)
        assert torch.equal(got[0], exp[0]) and torch.equal(got[1], exp[1])


def test_masked_attention_equals_attention_over_the_visible_keys_only():
    """Each query's row equals plain (unmasked) attention over just the keys it may see, gathered by
    hand from the padding row and the window; a query that sees none gets a zero row, LSE -inf."""
    q, k, v = rn(2, 2, 6, 8, seed=10), rn(2, 1, 10, 8, seed=11), rn(2, 1, 10, 8, seed=12)
    key_valid = torch.tensor([[0, 0, 0, 0, 0, 0, 1, 1, 1, 1], [1, 0, 1, 1, 0, 1, 1, 1, 0, 1]])
    off, win = 4, 3
    out, lse = O.attention_masked(q, k, v, 0.5, 2, off, key_valid, win)
    for b in range(2):
        for h in range(2):
            for i in range(6):
                vis = [j for j in range(10) if i + off - win < j <= i + off and key_valid[b, j]]
                if not vis:
                    assert torch.all(out[b, h, i] == 0) and lse[b, h, i] == float("-inf")
                    continue
                s = (q[b, h, i].double() @ k[b, 0, vis].double().T) * 0.5
                torch.testing.assert_close(out[b, h, i], torch.softmax(s, 0) @ v[b, 0, vis].double())
                torch.testing.assert_close(lse[b, h, i], torch.logsumexp(s, 0))
    assert (lse == float("-inf")).any()  # batch row 0, queries 0 and 1 see only padding


@pytest.mark.parametrize("causal,groups,off", [(True, 2, 0), (False, 1, 0), (True, 1, 3)])
def test_attention_backward_matches_autograd(causal, groups, off):
    q = rn(1, 4, 6, 8, seed=7).requires_grad_(True)
    k = rn(1, 4 // groups, 6 + off, 8, seed=8).requires_grad_(True)
    v = rn(1, 4 // groups, 6 + off, 8, seed=9).requires_grad_(True)
    go = rn(1, 4, 6, 8, seed=10)
    ke, ve = k.repeat_interleave(groups, 1), v.repeat_interleave(groups, 1)
    mask = None
    if causal:
        mask = torch.tensor([[j <= i + off for j in range(6 + off)] for i in range(6)])
    F.scaled_dot_product_attention(q, ke, ve, attn_mask=mask, scale=0.4).backward(go)
    dq, dk, dv = O.attention_backward(q, k, v, go, 0.4, causal, groups, off)
    torch.testing.assert_close(dq, q.grad)
    torch.testing.assert_close(dk, k.grad)
    torch.testing.assert_close(dv, v.grad)


# ---------------------------------------------------------------- RMSNorm
def test_rmsnorm_matches_hf_qwen3():
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    x = rn(3, 5, 64, seed=11, dtype=torch.float32)
    norm = Qwen3RMSNorm(64, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(rn(64, seed=12, dtype=torch.float32))
    torch.testing.assert_close(O.rmsnorm(x, norm.weight, 1e-6).float(), norm(x), atol=1e-6, rtol=1e-5)


def test_rmsnorm_one_plus_matches_hf_qwen3_next():
    """The one_plus branch (weight stored as w, applied as 1 + w) against HF's Qwen3-Next RMSNorm,
    an independent implementation of that form: forward, and the input and weight gradients
    of the oracle's closed-form backward against autograd through the HF module."""
    from transformers.models.qwen3_next.modeling_qwen3_next import Qwen3NextRMSNorm

    x = rn(3, 5, 64, seed=16, dtype=torch.float32).requires_grad_(True)
    go = rn(3, 5, 64, seed=18, dtype=torch.float32)
    norm = Qwen3NextRMSNorm(64, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(0.3 * rn(64, seed=17, dtype=torch.float32))
    y = norm(x)
    y.backward(go)
    torch.testing.assert_close(O.rmsnorm(x.detach(), norm.weight.detach(), 1e-6, one_plus=True).float(), y.detach(),
                               atol=1e-6, rtol=1e-5)
    gx, gw = O.rmsnorm_backward(x.detach(), norm.weight.detach(), go, 1e-6, one_plus=True)
    torch.testing.assert_close(gx.float(), x.grad, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(gw.float(), norm.weight.grad, atol=1e-5, rtol=1e-5)
    # without the offset the same weights give a different result (the branch is live)
    assert (O.rmsnorm(x.detach(), norm.weight.detach(), 1e-6).float() - y.detach()).abs().max() > 0.1


@pytest.mark.parametrize("one_plus", [False, True])
def test_rmsnorm_backward_matches_autograd(one_plus):
    x = rn(4, 7, 32, seed=13).requires_grad_(True)
    w = rn(32, seed=14).requires_grad_(True)
    go = rn(4, 7, 32, seed=15)
    y = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * (w + (1.0 if one_plus else 0.0))
    y.backward(go)
    gx, gw = O.rmsnorm_backward(x, w, go, 1e-6, one_plus)
    torch.testing.assert_close(gx, x.grad)
    torch.testing.assert_close(gw, w.grad)
    torch.testing.assert_close(O.rmsnorm(x, w, 1e-6, one_plus), y)


# ---------------------------------------------------------------- RoPE
def test_rope_full_rotary_matches_hf():
    from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb

    q, k = rn(2, 4, 6, 32, seed=16), rn(2, 2, 6, 32, seed=17)
    cos, sin = O.rotary_tables(torch.arange(6), 32, 1e6, D64)
    hq, hk = apply_rotary_pos_emb(q, k, cos, sin)
    torch.testing.assert_close(O.rope(q, cos, sin), hq)
    torch.testing.assert_close(O.rope(k, cos, sin), hk)


def test_rope_partial_is_complex_rotation():
    x = rn(2, 3, 5, 16, seed=18)
    cos, sin = rn(2, 5, 8, seed=19), rn(2, 5, 8, seed=20)  # arbitrary tables, as the reference test uses
    out = O.rope(x, cos, sin)
    z = torch.complex(x[..., :4], x[..., 4:8]) * torch.complex(cos[:, None, :, :4], sin[:, None, :, :4])
    torch.testing.assert_close(out[..., :4], z.real)
    torch.testing.assert_close(out[..., 4:8], z.imag)
    torch.testing.assert_close(out[..., 8:], x[..., 8:])


def test_rope_backward_is_adjoint():
    x, gr = rn(2, 3, 5, 16, seed=21), rn(2, 3, 5, 16, seed=22)
    cos, sin = rn(1, 5, 12, seed=23), rn(1, 5, 12, seed=24)
    lhs = (O.rope(x, cos, sin) * gr).sum()
    rhs = (x * O.rope_backward(gr, cos, sin)).sum()
    torch.testing.assert_close(lhs, rhs)


# ---------------------------------------------------------------- gated products
def test_gated_products_match_torch_and_autograd():
    a = rn(5, 33, seed=25).requires_grad_(True)
    b = rn(5, 33, seed=26).requires_grad_(True)
    go = rn(5, 33, seed=27)
    y = F.silu(a) * b
    torch.testing.assert_close(O.silu_mul(a, b), y)
    y.backward(go)
    ga, gb = O.silu_mul_backward(a, b, go)
    torch.testing.assert_close(ga, a.grad)
    torch.testing.assert_close(gb, b.grad)
    a.grad = b.grad = None
    y = a * torch.sigmoid(b)
    torch.testing.assert_close(O.sigmoid_mul(a, b), y)
    y.backward(go)
    ga, gb = O.sigmoid_mul_backward(a, b, go)
    torch.testing.assert_close(ga, a.grad)
    torch.testing.assert_close(gb, b.grad)


# ---------------------------------------------------------------- CE / softmax
def test_cross_entropy_matches_torch():
    x = rn(9, 37, seed=28).requires_grad_(True)
    t = torch.randint(0, 37, (9,), generator=g(29))
    t[[2, 5]] = -100
    ref = F.cross_entropy(x, t, ignore_index=-100)
    loss, lse, rows = O.cross_entropy(x, t)
    torch.testing.assert_close(loss, ref)
    torch.testing.assert_close(lse, torch.logsumexp(x, -1))
    (ref * 3.0).backward()
    torch.testing.assert_close(O.cross_entropy_backward(x, t, 3.0), x.grad)


def test_cross_entropy_all_ignored_clamps_to_zero():
    # reference kernel path divides by n_valid.clamp(min=1) (cross_entropy.py:157-160)
    x, t = rn(3, 5, seed=30), torch.full((3,), -100)
    assert float(O.cross_entropy(x, t)[0]) == 0.0


def test_softmax_matches_torch_and_autograd():
    x = rn(6, 19, seed=31).requires_grad_(True)
    y = torch.softmax(x, -1)
    torch.testing.assert_close(O.softmax(x), y)
    go = rn(6, 19, seed=32)
    y.backward(go)
    torch.testing.assert_close(O.softmax_backward(y, go), x.grad)


# ---------------------------------------------------------------- routing
def test_topk_matches_torch_on_distinct_values():
    x = rn(50, 128, seed=33, dtype=torch.float32)
    v, i = O.topk(x, 8)
    tv, ti = torch.topk(x, 8)
    assert torch.equal(i, ti) and torch.equal(v, tv)


def test_topk_tie_rule_lowest_index_first():
    x = torch.tensor([[1.0, 3.0, 3.0, 0.5, 3.0, 1.0], [2.0] * 6])
    assert O.topk(x, 4)[1].tolist() == [[1, 2, 4, 0], [0, 1, 2, 3]]


def test_one_hot_and_index_add_match_torch():
    idx = torch.randint(0, 11, (7, 3), generator=g(34))
    assert torch.equal(O.one_hot(idx, 11), F.one_hot(idx, 11))
    tgt, src = rn(10, 4, seed=35), rn(25, 4, seed=36)
    index = torch.randint(0, 10, (25,), generator=g(37))
    torch.testing.assert_close(O.index_add(tgt, src, index), tgt.clone().index_add_(0, index, src))


# ---------------------------------------------------------------- embedding / linear / cache
def test_embedding_and_backward_match_autograd():
    w = rn(20, 6, seed=38).requires_grad_(True)
    ids = torch.randint(0, 20, (3, 9), generator=g(39))
    y = F.embedding(ids, w, padding_idx=4)
    torch.testing.assert_close(O.embedding(ids, w), y)
    go = rn(3, 9, 6, seed=40)
    y.backward(go)
    torch.testing.assert_close(O.embedding_backward(ids, go, 20, padding_idx=4), w.grad)


def test_linear_and_backward_match_autograd():
    x = rn(2, 5, 7, seed=41).requires_grad_(True)
    w = rn(3, 7, seed=42).requires_grad_(True)
    b = rn(3, seed=43).requires_grad_(True)
    y = F.linear(x, w, b)
    torch.testing.assert_close(O.linear(x, w, b), y)
    go = rn(2, 5, 3, seed=44)
    y.backward(go)
    gx, gw, gb = O.linear_backward(x, w, go, need_bias=True)
    torch.testing.assert_close(gx, x.grad)
    torch.testing.assert_close(gw, w.grad)
    torch.testing.assert_close(gb, b.grad)


def test_kv_write_known_answer():
    # reference tests/test_kernels.py:181-189
    cache = torch.zeros(2, 3, 16, 8)
    values = rn(2, 3, 5, 8, seed=45, dtype=torch.float32)
    out = O.kv_write(cache, values, torch.tensor([0, 1, 4, 7, 8]))
    for s, p in enumerate([0, 1, 4, 7, 8]):
        assert torch.equal(out[:, :, p], values[:, :, s])
    untouched = [p for p in range(16) if p not in (0, 1, 4, 7, 8)]
    assert torch.count_nonzero(out[:, :, untouched]) == 0


# ---------------------------------------------------------------- MoE block vs HF
def test_moe_block_matches_hf_qwen3_moe():
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock

    torch.manual_seed(0)
    cfg = Qwen3MoeConfig(hidden_size=32, moe_intermediate_size=16, num_experts=6, num_experts_per_tok=2,
                         norm_topk_prob=True)
    blk = Qwen3MoeSparseMoeBlock(cfg).double()
    with torch.no_grad():
        for p in blk.parameters():
            p.copy_(torch.randn(p.shape, generator=g(46), dtype=D64) * 0.2)
    x = rn(2, 7, 32, seed=47)
    ref = blk(x)
    gu, dn = blk.experts.gate_up_proj, blk.experts.down_proj
    out, *_ = O.moe_block(x.view(-1, 32), blk.gate.weight, gu[:, :16], gu[:, 16:], dn, 2, True)
    torch.testing.assert_close(out.view(2, 7, 32), ref)


def test_moe_block_grads_match_hf_qwen3_moe_autograd():
    """The oracle's MoE gradients (input, router, every expert weight) against autograd through HF's
    Qwen3MoeSparseMoeBlock (transformers 5.15, fused expert layout) on shared fp64 weights."""
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock

    torch.manual_seed(0)
    I = 16
    cfg = Qwen3MoeConfig(hidden_size=32, moe_intermediate_size=I, num_experts=6, num_experts_per_tok=2,
                         norm_topk_prob=True)
    blk = Qwen3MoeSparseMoeBlock(cfg).double()
    with torch.no_grad():
        for p in blk.parameters():
            p.copy_(torch.randn(p.shape, generator=g(52), dtype=D64) * 0.3)
    x = rn(2, 9, 32, seed=53).requires_grad_(True)
    gout = rn(2, 9, 32, seed=54)
    ref = blk(x)
    (ref * gout).sum().backward()
    gu, dn = blk.experts.gate_up_proj, blk.experts.down_proj
    out, dx, dgw, dwg, dwu, dwd = O.moe_block_grads(x.view(-1, 32), blk.gate.weight, gu[:, :I], gu[:, I:], dn, 2,
                                                    gout.view(-1, 32), True)
    tol = dict(atol=1e-6, rtol=1e-5)  # HF takes the router softmax in fp32 even for fp64 weights
    torch.testing.assert_close(out.view(2, 9, 32), ref.detach(), **tol)
    torch.testing.assert_close(dx.view(2, 9, 32), x.grad, **tol)
    torch.testing.assert_close(dgw, blk.gate.weight.grad, **tol)
    torch.testing.assert_close(dwg, blk.experts.gate_up_proj.grad[:, :I], **tol)
    torch.testing.assert_close(dwu, blk.experts.gate_up_proj.grad[:, I:], **tol)
    torch.testing.assert_close(dwd, blk.experts.down_proj.grad, **tol)
    assert dgw.abs().max() > 1e-3  # the router path carries gradient


def test_kv_append_and_residual_add():
    a, b = rn(2, 3, 4, 5, seed=48), rn(2, 3, 2, 5, seed=49)
    out = O.kv_append(a, b)
    assert out.shape == (2, 3, 6, 5)
    assert torch.equal(out[:, :, :4], a) and torch.equal(out[:, :, 4:], b)
    x, r = rn(7, seed=50), rn(7, seed=51)
    assert torch.equal(O.residual_add(x, r), torch.add(x, r))


def test_gated_delta_rule_matches_hf_recurrent_and_chunked_forms():
    """The oracle's recurrence against transformers 5.15's torch_recurrent_gated_delta_rule and
    torch_chunk_gated_delta_rule (Qwen3-Next) in fp64, with and without an initial state."""
    from transformers.models.qwen3_next import modeling_qwen3_next as M

    B, S, H, K, V = 2, 37, 3, 16, 8
    # L2-normalised q and k, as the model feeds them (the update I - beta k k^T is then a contraction;
    # HF evaluates in fp32 whatever the input dtype, hence the fp32 band)
    q, k, v = rn(B, S, H, K, seed=60), rn(B, S, H, K, seed=61), rn(B, S, H, V, seed=62)
    q, k = q / q.norm(dim=-1, keepdim=True), k / k.norm(dim=-1, keepdim=True)
    g = -rn(B, S, H, seed=63).abs() * 0.3
    beta = torch.sigmoid(rn(B, S, H, seed=64))
    s0 = rn(B, H, K, V, seed=65)
    for init in (None, s0):
        out, st = O.gated_delta_rule(q, k, v, g, beta, init)
        ho, hs = M.torch_recurrent_gated_delta_rule(q, k, v, g=g, beta=beta, initial_state=init,
                                                    output_final_state=True)
        f32 = dict(atol=2e-5, rtol=2e-5)
        torch.testing.assert_close(out, ho.double(), **f32)
        torch.testing.assert_close(st, hs.double(), **f32)
        co, cs = M.torch_chunk_gated_delta_rule(q, k, v, g=g, beta=beta, initial_state=init,
                                                output_final_state=True)
        torch.testing.assert_close(out, co.double(), **f32)
        torch.testing.assert_close(st, cs.double(), **f32)


def test_gated_delta_rule_closed_form_single_token():
    """One token from a zero state: S = beta k v^T, so o = beta (q.k) v / sqrt(K) for every head."""
    q, k, v = rn(1, 1, 2, 4, seed=66), rn(1, 1, 2, 4, seed=67), rn(1, 1, 2, 3, seed=68)
    g, beta = rn(1, 1, 2, seed=69), torch.sigmoid(rn(1, 1, 2, seed=70))
    out, st = O.gated_delta_rule(q, k, v, g, beta)
    expect = beta[..., None] * (q * k).sum(-1, keepdim=True) * v / 2.0
    torch.testing.assert_close(out, expect)
    torch.testing.assert_close(st[0, 0], beta[0, 0, 0] * torch.outer(k[0, 0, 0], v[0, 0, 0]))
