"""CPU restatement of the reference operator semantics (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this module, and only as the checker. Every function evaluates in
float64 on the CPU (unless a dtype is passed) and cites the reference code it
restates (paths relative to the luozoupi/Qwen-Triton checkout).

Each function is pinned by ``tests/test_oracle.py`` against an independent
authority: torch built-ins (SDPA, cross_entropy, softmax, topk, index_add_,
one_hot, embedding), autograd of the forward formulas, the HF transformers
implementation of Qwen3 (``apply_rotary_pos_emb``, ``Qwen3RMSNorm``), algebraic
identities (RoPE adjointness, softmax rows summing to one) and the reference's
own known-answer test for the KV write.
"""
from __future__ import annotations

import torch

F64 = torch.float64


def _d(t: torch.Tensor, dtype=F64) -> torch.Tensor:
    return t.detach().to("cpu", dtype)


# ---------------------------------------------------------------------------
# Linear — qwen_triton/kernels/matmul.py:35-49 (torch restatement of :130-200)
# ---------------------------------------------------------------------------
def linear(x, weight, bias=None, dtype=F64):
    y = _d(x, dtype) @ _d(weight, dtype).T
    if bias is not None:
        y = y + _d(bias, dtype)
    return y


def linear_backward(x, weight, grad_out, need_bias=False, dtype=F64):
    g = _d(grad_out, dtype)
    g2 = g.reshape(-1, g.shape[-1])
    x2 = _d(x, dtype).reshape(-1, x.shape[-1])
    gx = (g2 @ _d(weight, dtype)).reshape(*g.shape[:-1], weight.shape[1])
    gw = g2.T @ x2
    gb = g2.sum(0) if need_bias else None
    return gx, gw, gb


# ---------------------------------------------------------------------------
# Embedding — qwen_triton/kernels/embedding.py:35-36 (forward), :146-163 (backward)
# ---------------------------------------------------------------------------
def embedding(ids, weight, dtype=F64):
    return _d(weight, dtype)[ids.cpu().long()]


def embedding_backward(ids, grad_out, num_embeddings, padding_idx=None, dtype=F64):
    flat = ids.cpu().long().reshape(-1)
    g = _d(grad_out, dtype).reshape(flat.numel(), -1)
    gw = torch.zeros((num_embeddings, g.shape[1]), dtype=dtype)
    for t in range(flat.numel()):  # token order, as the sum is defined
        gw[flat[t]] += g[t]
    if padding_idx is not None:
        gw[padding_idx] = 0
    return gw


# ---------------------------------------------------------------------------
# Attention — qwen_triton/kernels/flash_attention.py:35-49 (SDPA restatement of
# the kernels :54-277); causal key j visible to query i iff j <= i + offset.
# ---------------------------------------------------------------------------
def _expand_kv(k, groups):
    return k.repeat_interleave(groups, dim=1) if groups > 1 else k


def attention(q, k, v, scale, causal=True, groups=1, causal_offset=0, dtype=F64):
    """Returns (out [B,Hq,Sq,D], lse [B,Hq,Sq]) by brute force."""
    q, k, v = _d(q, dtype), _expand_kv(_d(k, dtype), groups), _expand_kv(_d(v, dtype), groups)
    s = (q @ k.transpose(-1, -2)) * scale
    if causal:
        sq, sk = s.shape[-2], s.shape[-1]
        allowed = torch.arange(sk)[None, :] <= torch.arange(sq)[:, None] + causal_offset
        s = s.masked_fill(~allowed, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse[..., None])
    p = torch.nan_to_num(p, nan=0.0)
    return p @ v, lse


def attention_masked(q, k, v, scale, groups=1, causal_offset=0, key_valid=None, window=None, dtype=F64):
    """Causal attention under the decoder's padding / sliding-window mask, by brute force: key j is
    visible to query i iff j <= i + causal_offset, j > i + causal_offset - window (window set) and
    key_valid[b, j] != 0 (qwen_triton/models/core.py:47-75 builds this mask, SDPA applies it at
    qwen_triton/modules/attention.py:114-119). Hidden keys get -inf, so a query that sees no key
    has a zero row and LSE -inf (the reference's finite additive mask gives such padding rows,
    whose outputs are never used, an average instead). Returns (out, lse)."""
    q, k, v = _d(q, dtype), _expand_kv(_d(k, dtype), groups), _expand_kv(_d(v, dtype), groups)
    s = (q @ k.transpose(-1, -2)) * scale
    sq, sk = s.shape[-2], s.shape[-1]
    pos = torch.arange(sq)[:, None] + causal_offset
    keys = torch.arange(sk)[None, :]
    allowed = keys <= pos
    if window is not None:
        allowed = allowed & (keys > pos - window)
    allowed = allowed[None, None].expand(s.shape[0], 1, sq, sk)
    if key_valid is not None:
        allowed = allowed & (key_valid.cpu() != 0)[:, None, None, :sk]
    s = s.masked_fill(~allowed, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.nan_to_num(torch.exp(s - lse[..., None]), nan=0.0)
    return p @ v, lse


def attention_backward(q, k, v, grad_out, scale, causal=True, groups=1, causal_offset=0, dtype=F64):
    """dq, dk, dv from the softmax-attention derivative (dk/dv summed over each GQA group)."""
    qd, kd, vd = _d(q, dtype), _expand_kv(_d(k, dtype), groups), _expand_kv(_d(v, dtype), groups)
    out, lse = attention(q, k, v, scale, causal, groups, causal_offset, dtype)
    s = (qd @ kd.transpose(-1, -2)) * scale
    p = torch.nan_to_num(torch.exp(s - lse[..., None]), nan=0.0)
    if causal:
        sq, sk = s.shape[-2], s.shape[-1]
        allowed = torch.arange(sk)[None, :] <= torch.arange(sq)[:, None] + causal_offset
        p = p * allowed
    do = _d(grad_out, dtype)
    dv = p.transpose(-1, -2) @ do
    dp = do @ vd.transpose(-1, -2)
    delta = (do * out).sum(-1, keepdim=True)
    ds = p * (dp - delta)
    dq = (ds @ kd) * scale
    dk = (ds.transpose(-1, -2) @ qd) * scale
    if groups > 1:
        B, H, S, D = dk.shape
        dk = dk.view(B, H // groups, groups, S, D).sum(2)
        dv = dv.view(B, H // groups, groups, S, D).sum(2)
    return dq, dk, dv


# ---------------------------------------------------------------------------
# RMSNorm — qwen_triton/kernels/rmsnorm.py:35-62
# ---------------------------------------------------------------------------
def rmsnorm(x, weight, eps=1e-6, one_plus=False, dtype=F64):
    xd = _d(x, dtype)
    w = _d(weight, dtype) + (1.0 if one_plus else 0.0)
    return xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps) * w


def rmsnorm_backward(x, weight, grad_out, eps=1e-6, one_plus=False, dtype=F64):
    xd, g = _d(x, dtype), _d(grad_out, dtype)
    w = _d(weight, dtype) + (1.0 if one_plus else 0.0)
    n = xd.shape[-1]
    inv = torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps)
    gw = (g * xd * inv).reshape(-1, n).sum(0)
    dot = (g * w * xd).sum(-1, keepdim=True)
    gx = g * w * inv - xd * inv.pow(3) * dot / n
    return gx, gw


# ---------------------------------------------------------------------------
# RoPE — qwen_triton/kernels/rope.py:59-73 (forward), :165-203 (backward = -sin)
# ---------------------------------------------------------------------------
def rope(x, cos, sin, dtype=F64):
    """x [B,H,S,D]; cos/sin [B or 1, S, rot]; uses cos/sin[..., :rot/2] only."""
    xd, c, s = _d(x, dtype), _d(cos, dtype), _d(sin, dtype)
    rot = c.shape[-1]
    half = rot // 2
    c = c[:, None, :, :half]
    s = s[:, None, :, :half]
    x1, x2, rest = xd[..., :half], xd[..., half:rot], xd[..., rot:]
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s, rest), dim=-1)


def rope_backward(grad_out, cos, sin, dtype=F64):
    return rope(grad_out, cos, -_d(sin, dtype), dtype)


# ---------------------------------------------------------------------------
# Gated products — qwen_triton/kernels/swiglu.py:35-51, sigmoid_mul.py:35-50
# ---------------------------------------------------------------------------
def silu_mul(gate, up, dtype=F64):
    g, u = _d(gate, dtype), _d(up, dtype)
    return g * torch.sigmoid(g) * u


def silu_mul_backward(gate, up, grad_out, dtype=F64):
    g, u, go = _d(gate, dtype), _d(up, dtype), _d(grad_out, dtype)
    s = torch.sigmoid(g)
    return go * u * s * (1 + g * (1 - s)), go * g * s


def sigmoid_mul(x, gate, dtype=F64):
    return _d(x, dtype) * torch.sigmoid(_d(gate, dtype))


def sigmoid_mul_backward(x, gate, grad_out, dtype=F64):
    xd, g, go = _d(x, dtype), _d(gate, dtype), _d(grad_out, dtype)
    s = torch.sigmoid(g)
    return go * s, go * xd * s * (1 - s)


def residual_add(x, r, dtype=F64):
    """qwen_triton/kernels/residual_add.py:35-36"""
    return _d(x, dtype) + _d(r, dtype)


# ---------------------------------------------------------------------------
# KV cache — qwen_triton/kernels/cache.py:142-181 (write), :101-139 (append)
# ---------------------------------------------------------------------------
def kv_write(cache, values, positions):
    out = cache.detach().cpu().clone()
    out[:, :, positions.cpu().long(), :] = values.detach().cpu().to(out.dtype)
    return out


def kv_append(prefix, suffix):
    return torch.cat((prefix.detach().cpu(), suffix.detach().cpu()), dim=-2)


# ---------------------------------------------------------------------------
# Cross-entropy — qwen_triton/kernels/cross_entropy.py:142-161 (mean over
# non-ignored rows, clamp(n_valid, 1)), backward :108-139
# ---------------------------------------------------------------------------
def cross_entropy(logits, targets, ignore_index=-100, dtype=F64):
    x, t = _d(logits, dtype), targets.cpu().long()
    lse = torch.logsumexp(x, dim=-1)
    valid = t != ignore_index
    picked = x.gather(1, t.clamp(0, x.shape[1] - 1)[:, None])[:, 0]
    rows = torch.where(valid, lse - picked, torch.zeros_like(lse))
    n = valid.sum().clamp(min=1)
    return rows.sum() / n, lse, rows


def cross_entropy_backward(logits, targets, grad_loss=1.0, ignore_index=-100, dtype=F64):
    x, t = _d(logits, dtype), targets.cpu().long()
    valid = t != ignore_index
    p = torch.softmax(x, dim=-1)
    onehot = torch.zeros_like(p)
    onehot[valid, t[valid]] = 1.0
    n = valid.sum().clamp(min=1)
    g = (p - onehot) * (float(grad_loss) / n)
    g[~valid] = 0
    return g


# ---------------------------------------------------------------------------
# Softmax — qwen_triton/kernels/softmax.py:35-41
# ---------------------------------------------------------------------------
def softmax(x, dtype=F64):
    xd = _d(x, dtype)
    e = torch.exp(xd - xd.max(dim=-1, keepdim=True).values)
    return e / e.sum(-1, keepdim=True)


def softmax_backward(y, grad_out, dtype=F64):
    yd, g = _d(y, dtype), _d(grad_out, dtype)
    return yd * (g - (g * yd).sum(-1, keepdim=True))


# ---------------------------------------------------------------------------
# MoE routing — qwen_triton/kernels/moe_routing.py:84-116 (top-k: descending,
# ties to the lowest index), :171-200 (one-hot), :207-255 (index_add)
# ---------------------------------------------------------------------------
def topk(x, k):
    """Exact selection rule by a stable sort on the negated values."""
    xd = x.detach().cpu()
    order = torch.sort(-xd.to(F64), dim=-1, stable=True).indices[:, :k]
    return xd.gather(1, order), order


def one_hot(idx, num_classes):
    flat = idx.cpu().long().reshape(-1)
    out = torch.zeros((flat.numel(), num_classes), dtype=torch.int64)
    for i, v in enumerate(flat.tolist()):
        if 0 <= v < num_classes:
            out[i, v] = 1
    return out.view(*idx.shape, num_classes)


def index_add(target, source, index, dtype=F64):
    out = _d(target, dtype).clone()
    src = _d(source, dtype)
    for r, t in enumerate(index.cpu().long().tolist()):
        if 0 <= t < out.shape[0]:
            out[t] += src[r]
    return out


# ---------------------------------------------------------------------------
# Sparse MoE block — qwen_triton/modules/moe.py:32-58
# ---------------------------------------------------------------------------
def moe_block(x, gate_w, w_gate, w_up, w_down, top_k, norm_topk_prob=True, router_logits=None, dtype=F64):
    """x [T,H]; gate_w [E,H]; w_gate/w_up [E,I,H]; w_down [E,H,I]. Returns (out, logits, weights, experts)."""
    xd = _d(x, dtype)
    logits = _d(router_logits, dtype) if router_logits is not None else xd @ _d(gate_w, dtype).T
    probs = softmax(logits, dtype)
    weights, experts = topk(probs, top_k)
    weights = weights.to(dtype)
    if norm_topk_prob:
        weights = weights / weights.sum(-1, keepdim=True)
    out = torch.zeros_like(xd)
    for e in range(w_gate.shape[0]):
        tok, slot = torch.where(experts == e)
        if tok.numel() == 0:
            continue
        xe = xd[tok]
        h = silu_mul(xe @ _d(w_gate[e], dtype).T, xe @ _d(w_up[e], dtype).T, dtype) @ _d(w_down[e], dtype).T
        out.index_add_(0, tok, h * weights[tok, slot, None])
    return out, logits, weights, experts


def moe_block_grads(x, gate_w, w_gate, w_up, w_down, top_k, grad_out, norm_topk_prob=True, dtype=F64,
                    experts=None):
    """Gradients of sum(moe_block(x, gate_w, ...) * grad_out) by autograd, through both the experts
    and the router (softmax, the selected probabilities, their renormalisation, the gate projection).
    The expert choice is the forward's top-k selection and carries no gradient itself, as in the
    reference, whose top-k backward scatters only into the selected entries
    (qwen_triton/kernels/moe_routing.py:147-162). ``experts`` [T, top_k] may fix that choice (a
    caller comparing against another evaluation whose near-ties could resolve differently).
    Returns (out, dx, dgate_w, dw_gate, dw_up, dw_down)."""
    leaves = [_d(t, dtype).requires_grad_(True) for t in (x, gate_w, w_gate, w_up, w_down)]
    xd, gw, wg, wu, wdn = leaves
    with torch.enable_grad():
        probs = torch.softmax(xd @ gw.T, dim=-1)
        experts = topk(probs, top_k)[1] if experts is None else experts.cpu().long()
        weights = probs.gather(1, experts)
        if norm_topk_prob:
            weights = weights / weights.sum(-1, keepdim=True)
        out = torch.zeros_like(xd)
        for e in range(wg.shape[0]):
            tok, slot = torch.where(experts == e)
            if tok.numel() == 0:
                continue
            xe = xd[tok]
            h = (torch.nn.functional.silu(xe @ wg[e].T) * (xe @ wu[e].T)) @ wdn[e].T
            out = out.index_add(0, tok, h * weights[tok, slot, None])
        (out * _d(grad_out, dtype)).sum().backward()
    return (out.detach(),) + tuple(t.grad for t in leaves)


# ---------------------------------------------------------------------------
# Gated delta rule — qwen_triton/kernels/linear_attention.py:35-51 (step) and :130-189 (sequence)
# ---------------------------------------------------------------------------
def gated_delta_rule(q, k, v, g, beta, initial_state=None, dtype=F64):
    """q/k [B,S,H,K], v [B,S,H,V], g/beta [B,S,H] -> (out [B,S,H,V], final state [B,H,K,V]).

    The query is scaled by K^-0.5 in its own dtype first (as the reference does), then, per token,
    S = S exp(g); d = (v - S^T k) beta; S += k d^T; o = S^T q."""
    B, S, H, K = q.shape
    q = (q * (K ** -0.5)).detach().to("cpu", dtype)
    k, v, g, beta = (_d(t, dtype) for t in (k, v, g, beta))
    st = torch.zeros(B, H, K, v.shape[-1], dtype=dtype) if initial_state is None else _d(initial_state, dtype)
    out = torch.zeros(B, S, H, v.shape[-1], dtype=dtype)
    for t in range(S):
        st = st * g[:, t].exp()[:, :, None, None]
        kv = (st * k[:, t, :, :, None]).sum(dim=-2)
        d = (v[:, t] - kv) * beta[:, t, :, None]
        st = st + k[:, t, :, :, None] * d[:, :, None, :]
        out[:, t] = (st * q[:, t, :, :, None]).sum(dim=-2)
    return out, st


def rotary_tables(positions, rotary_dim, theta, dtype=torch.float32):
    """cos/sin [1, S, rot] — qwen_triton/modules/rotary.py:10-26 (fp32 tables)."""
    inv = 1.0 / (theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))
    freqs = positions.cpu().to(torch.float32)[:, None] * inv[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)[None]
    return emb.cos().to(dtype), emb.sin().to(dtype)

