"""Parity at the full sizes of the benchmark configurations (configs 1-4).

At these sizes the CPU oracle would take minutes per op, so each test checks the HIP path
against one of:
- an fp32 torch evaluation of the same op on the GPU, for floating-point kernels (computed
  head by head or expert by expert to bound memory);
- the CPU oracle on a sample of independent sequences (the model's decode step);
- properties that do not depend on size (cross-entropy gradient rows summing to zero,
  bitwise-equal reruns).

Bands are relative to the reference tensor's largest magnitude, since these are sums over
thousands of bf16 products: max|ours - ref| <= tol * max|ref| + tol_abs.
"""
from __future__ import annotations

import pytest
import torch

from qwen_triton import kernels as K
from qwen_triton.kernels import flash_attention as FA

from _util import native_calls

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _randn(shape, seed, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=DEV) * scale).to(dtype)


def _rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    a, e = actual.detach().float(), expected.detach().float()
    return float((a - e).abs().max()) / max(float(e.abs().max()), 1e-12)


def _rms_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    a, e = actual.detach().double(), expected.detach().double()
    return float((a - e).norm()) / max(float(e.norm()), 1e-300)


_STATS: dict[str, tuple[float, float]] = {}


def _check(actual, expected, tol, what, rms_tol=None):
    """max|diff| / max|ref| <= tol and, when given, the relative RMS error ||diff|| / ||ref|| <= rms_tol
    (the second bounds the bulk of the elements, small ones included)."""
    err, rms = _rel_err(actual, expected), _rms_err(actual, expected)
    _STATS[what] = (err, rms)
    print(f"[fullsize] {what}: max-rel {err:.3e} rms-rel {rms:.3e}", flush=True)
    assert err <= tol, f"{what}: max|diff| / max|ref| = {err:.3e} > {tol}"
    if rms_tol is not None:
        assert rms <= rms_tol, f"{what}: ||diff|| / ||ref|| = {rms:.3e} > {rms_tol}"


# ---------------------------------------------------------------------------
# config 1: flash attention forward + backward, 8 x 16 q-heads / 8 kv-heads x 4096 x 128, causal
# ---------------------------------------------------------------------------
def test_flash_attention_config1_full_size():
    B, Hq, Hkv, S, D = 8, 16, 8, 4096, 128
    G = Hq // Hkv
    scale = D ** -0.5
    q, k, v, do = _randn((B, Hq, S, D), 1), _randn((B, Hkv, S, D), 2), _randn((B, Hkv, S, D), 3), \
        _randn((B, Hq, S, D), 4)
    cf, cb = native_calls("qh_flash_fwd"), native_calls("qh_flash_bwd")
    o, lse = FA.flash_forward(q, k, v, scale, True, G)
    dq, dk, dv = FA.flash_backward(q, k, v, o, do, lse, scale, True, G)
    assert native_calls("qh_flash_fwd") == cf + 1 and native_calls("qh_flash_bwd") == cb + 1
    # determinism of the whole pass
    o2, lse2 = FA.flash_forward(q, k, v, scale, True, G)
    dq2, dk2, dv2 = FA.flash_backward(q, k, v, o2, do, lse2, scale, True, G)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    assert torch.equal(dq, dq2) and torch.equal(dk, dk2) and torch.equal(dv, dv2)

    visible = torch.ones(S, S, dtype=torch.bool, device=DEV).tril()
    dk_ref = torch.zeros(B, Hkv, S, D, device=DEV)
    dv_ref = torch.zeros(B, Hkv, S, D, device=DEV)
    worst = {"o": 0.0, "lse": 0.0, "dq": 0.0}
    for b in range(B):
        for h in range(Hq):
            hk = h // G
            qf, kf, vf, dof = q[b, h].float(), k[b, hk].float(), v[b, hk].float(), do[b, h].float()
            s = (qf @ kf.t().contiguous()) * scale
            s.masked_fill_(~visible, float("-inf"))
            lse_ref = torch.logsumexp(s, dim=-1)
            p = torch.exp(s - lse_ref[:, None])
            o_ref = p @ vf
            dp = dof @ vf.t().contiguous()
            ds = p * (dp - (dof * o_ref).sum(-1, keepdim=True))
            worst["o"] = max(worst["o"], _rel_err(o[b, h], o_ref))
            worst["o_rms"] = max(worst.get("o_rms", 0.0), _rms_err(o[b, h], o_ref))
            worst["lse"] = max(worst["lse"], float((lse[b, h] - lse_ref).abs().max()))
            dq_ref = (ds @ kf) * scale
            worst["dq"] = max(worst["dq"], _rel_err(dq[b, h], dq_ref))
            worst["dq_rms"] = max(worst.get("dq_rms", 0.0), _rms_err(dq[b, h], dq_ref))
            dk_ref[b, hk] += (ds.t().contiguous() @ qf) * scale
            dv_ref[b, hk] += p.t().contiguous() @ dof
    print(f"[fullsize] config1 worst per head: {worst}", flush=True)
    assert worst["o"] <= 2e-2 and worst["o_rms"] <= 5e-3, worst
    assert worst["lse"] <= 1e-3, worst
    assert worst["dq"] <= 2e-2 and worst["dq_rms"] <= 6e-3, worst
    for b in range(B):
        for hk in range(Hkv):
            _check(dk[b, hk], dk_ref[b, hk], 2e-2, f"dk[{b},{hk}]", rms_tol=6e-3)
            _check(dv[b, hk], dv_ref[b, hk], 2e-2, f"dv[{b},{hk}]", rms_tol=6e-3)


# ---------------------------------------------------------------------------
# config 3: decode attention, 64 sequences x 2049 cached keys (cache capacity 2112)
# ---------------------------------------------------------------------------
def test_decode_attention_config3_full_size():
    B, Hq, Hkv, D, cap, Sk = 64, 16, 8, 128, 2112, 2049
    G = Hq // Hkv
    scale = D ** -0.5
    kc, vc, q = _randn((B, Hkv, cap, D), 11), _randn((B, Hkv, cap, D), 12), _randn((B, Hq, 1, D), 13)
    lens = torch.randint(1, Sk + 1, (B,), generator=torch.Generator().manual_seed(14)).to(torch.int32).to(DEV)
    c0 = native_calls("qh_flash_decode")
    out = FA.flash_decode(q, kc[:, :, :Sk], vc[:, :, :Sk], scale, G)
    out_l = FA.flash_decode(q, kc[:, :, :Sk], vc[:, :, :Sk], scale, G, seqlens=lens)
    assert native_calls("qh_flash_decode") == c0 + 2
    assert torch.equal(out, FA.flash_decode(q, kc[:, :, :Sk], vc[:, :, :Sk], scale, G))

    qf = q.float().view(B, Hkv, G, D)
    kf, vf = kc[:, :, :Sk].float(), vc[:, :, :Sk].float()
    s = (qf @ kf.transpose(-1, -2).contiguous()) * scale  # [B, Hkv, G, Sk]
    ref = (torch.softmax(s, dim=-1) @ vf).view(B, Hq, 1, D)
    _check(out, ref, 2e-2, "decode", rms_tol=5e-3)
    keep = torch.arange(Sk, device=DEV)[None, :] < lens[:, None].long()  # [B, Sk]
    s_l = s.masked_fill(~keep[:, None, None, :], float("-inf"))
    ref_l = (torch.softmax(s_l, dim=-1) @ vf).view(B, Hq, 1, D)
    _check(out_l, ref_l, 2e-2, "decode with seqlens", rms_tol=5e-3)


# ---------------------------------------------------------------------------
# config 2: gate/up + SiLU-mul + down, LM head and cross-entropy on 16384 tokens, fwd + bwd
# ---------------------------------------------------------------------------
def test_dense_block_config2_full_size():
    T, H, I, V = 16384, 1024, 3072, 151936
    x = _randn((T, H), 21).requires_grad_(True)
    wg, wu, wd = (_randn(sh, sd, scale=0.02).requires_grad_(True) for sh, sd in (((I, H), 22), ((I, H), 23),
                                                                                 ((H, I), 24)))
    wl = _randn((V, H), 25, scale=0.02).requires_grad_(True)
    labels = torch.randint(0, V, (T,), generator=torch.Generator().manual_seed(26)).to(DEV)
    c_mm, c_ce = native_calls("qh_gemm"), native_calls("qh_ce_fwd")
    y = K.triton_matmul(K.silu_mul(K.triton_matmul(x, wg), K.triton_matmul(x, wu)), wd)
    logits = K.triton_matmul(y, wl)
    logits.retain_grad()
    loss = K.triton_cross_entropy(logits, labels)
    loss.backward()
    assert native_calls("qh_gemm") > c_mm and native_calls("qh_ce_fwd") > c_ce
    # each cross-entropy gradient row is softmax - one-hot, scaled: it sums to zero
    g = logits.grad.float()
    assert float(g.sum(-1).abs().max()) <= 1e-3 * float(g.abs().max())

    xr, wgr, wur, wdr, wlr = (t.detach().float().requires_grad_(True) for t in (x, wg, wu, wd, wl))
    gr = xr @ wgr.t()
    yr = (torch.nn.functional.silu(gr) * (xr @ wur.t())) @ wdr.t()
    lr = yr @ wlr.t()
    loss_r = torch.nn.functional.cross_entropy(lr, labels)
    loss_r.backward()
    assert abs(float(loss) - float(loss_r)) <= 2e-3 * abs(float(loss_r))
    _check(y, yr, 2e-2, "down output", rms_tol=1e-2)
    _check(logits, lr, 2e-2, "logits", rms_tol=1e-2)
    for name, a, r in (("x", x, xr), ("gate", wg, wgr), ("up", wu, wur), ("down", wd, wdr), ("lm_head", wl, wlr)):
        _check(a.grad, r.grad, 3e-2, f"d{name}", rms_tol=1e-2)


# ---------------------------------------------------------------------------
# config 4: MoE experts (128 experts, top-8, hidden 2048, intermediate 768) on 16384 tokens
# ---------------------------------------------------------------------------
def _moe_block_config4():
    from qwen_triton import QwenTritonConfig
    from qwen_triton.modules import QwenSparseMoeBlock

    cfg = QwenTritonConfig.from_hf_config(dict(
        model_type="qwen3_moe", vocab_size=64, hidden_size=2048, intermediate_size=6144, num_hidden_layers=1,
        num_attention_heads=32, num_key_value_heads=4, head_dim=128, moe_intermediate_size=768, num_experts=128,
        num_experts_per_tok=8, norm_topk_prob=True, decoder_sparse_step=1, mlp_only_layers=[]))
    torch.manual_seed(0)
    blk = QwenSparseMoeBlock(cfg)
    with torch.no_grad():
        for p in blk.parameters():
            p.normal_(0.0, 0.02)
    return blk.to(DEV, torch.bfloat16)


def test_moe_experts_config4_full_size():
    blk = _moe_block_config4()
    T, H = 16384, 2048
    x0 = _randn((T, H), 31)
    logits = _randn((T, 128), 32, dtype=torch.float32)
    go = _randn((T, H), 33, scale=0.01)
    w, sel = blk.route(logits, torch.bfloat16)
    weights = [p for e in blk.experts for p in (e.gate_proj.weight, e.up_proj.weight, e.down_proj.weight)]

    def loop():
        saved = blk._grouped_ok
        blk._grouped_ok = lambda *a, **kw: False
        try:
            return blk.experts_forward(x, w, sel)
        finally:
            blk._grouped_ok = saved

    c_up = native_calls("qh_moe_up")
    with torch.no_grad():
        x = x0
        inf = blk.experts_forward(x0, w, sel)
        ref_inf = loop()
    assert native_calls("qh_moe_up") == c_up + 1
    _check(inf, ref_inf, 2e-2, "inference forward", rms_tol=2e-3)

    def run(grouped):
        nonlocal x
        x = x0.clone().requires_grad_(True)
        for p in weights:
            p.grad = None
        out = blk.experts_forward(x, w, sel) if grouped else loop()
        out.backward(go)
        return out.detach(), x.grad.clone(), [p.grad.clone() for p in weights]

    out, gx, gw = run(True)
    rout, rgx, rgw = run(False)
    assert torch.equal(out, inf)  # the training forward is the inference forward plus saved G, U
    _check(out, rout, 2e-2, "training forward", rms_tol=2e-3)
    _check(gx, rgx, 2e-2, "d input", rms_tol=1.5e-2)
    worst = max(_rel_err(a, b) for a, b in zip(gw, rgw))
    assert worst <= 3e-2, f"expert weight gradients: {worst:.3e}"

    # the reference's expert loop (modules/moe.py:32-58: per expert, SwiGLU on its tokens' rows,
    # times the routing weight, index_add into the output) in fp32 torch, with autograd
    xr = x0.detach().float().requires_grad_(True)
    wr = [p.detach().float().requires_grad_(True) for p in weights]
    acc = torch.zeros((T, H), dtype=torch.float32, device=DEV)
    wf = w.float()
    for e in range(len(blk.experts)):
        tok, slot = (sel == e).nonzero(as_tuple=True)
        if tok.numel() == 0:
            continue
        g_w, u_w, d_w = wr[3 * e], wr[3 * e + 1], wr[3 * e + 2]
        h = xr[tok]
        y = (torch.nn.functional.silu(h @ g_w.t()) * (h @ u_w.t())) @ d_w.t()
        acc = acc.index_add(0, tok, y * wf[tok, slot, None])
    acc.backward(go.float())
    _check(out, acc, 2e-2, "training forward vs fp32 loop", rms_tol=1.2e-2)
    _check(gx, xr.grad, 2e-2, "d input vs fp32 loop", rms_tol=1.2e-2)
    worst_f32, worst_rms = 0.0, 0.0
    for a, r in zip(gw, wr):
        if r.grad is None:  # an expert without tokens: exact zeros
            assert not bool(a.any()), "expert without tokens has a nonzero weight gradient"
            continue
        worst_f32, worst_rms = max(worst_f32, _rel_err(a, r.grad)), max(worst_rms, _rms_err(a, r.grad))
    print(f"[fullsize] config4 expert weight gradients vs fp32 loop: max-rel {worst_f32:.3e} rms-rel {worst_rms:.3e}",
          flush=True)
    assert worst_f32 <= 3e-2 and worst_rms <= 1.2e-2, f"expert weight gradients vs fp32 loop: {worst_f32:.3e}"


# ---------------------------------------------------------------------------
# config 3: the model's decode step (64 sequences, 2048 cached positions) vs the CPU oracle
# ---------------------------------------------------------------------------
def test_model_decode_step_config3_full_size():
    from oracle.model import ModelSpec, OracleQwen
    from qwen_triton import QwenTritonConfig, QwenTritonForCausalLM

    cfg = QwenTritonConfig.from_hf_config(dict(
        model_type="qwen3", vocab_size=151936, hidden_size=1024, intermediate_size=3072, num_hidden_layers=28,
        num_attention_heads=16, num_key_value_heads=8, head_dim=128, max_position_embeddings=40960,
        rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True))
    torch.manual_seed(0)
    model = QwenTritonForCausalLM(cfg, init_weights=False)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, 0.02)
    model = model.to(DEV, torch.bfloat16).eval()
    B, ctx = 64, 2048
    cache = model.new_cache(B, ctx + 64, torch.bfloat16, DEV)
    gen = torch.Generator(device=DEV).manual_seed(41)
    for i in range(cfg.num_hidden_layers):
        cache.key_cache[i][:, :, :ctx].normal_(generator=gen)
        cache.value_cache[i][:, :, :ctx].normal_(generator=gen)
        cache.attention_lengths[i] = ctx
    ids = torch.randint(0, cfg.vocab_size, (B, 1), generator=torch.Generator().manual_seed(42)).to(DEV)
    sample = [0, 37]
    kv = [(cache.key_cache[i][sample, :, :ctx].float().cpu(), cache.value_cache[i][sample, :, :ctx].float().cpu())
          for i in range(cfg.num_hidden_layers)]
    with torch.no_grad():
        logits = model(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=1).logits[:, -1]
    params = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    orc = OracleQwen(ModelSpec.from_config(cfg), params, dtype=torch.float32)
    ref = orc.forward(ids[sample].cpu(), {"k": [a for a, _ in kv], "v": [b for _, b in kv], "len": ctx},
                      logits_to_keep=1)[:, -1]
    got = logits[sample].float().cpu()
    # bf16 rounding over 28 layers at position 2048: the band is calibrated by the oracle itself
    # run in bf16 (the model's precision) against its fp32 run on the same weights and cache
    orc16 = OracleQwen(ModelSpec.from_config(cfg), params, dtype=torch.bfloat16)
    ref16 = orc16.forward(ids[sample].cpu(), {"k": [a.bfloat16() for a, _ in kv], "v": [b.bfloat16() for _, b in kv],
                                              "len": ctx}, logits_to_keep=1)[:, -1].float()
    noise = float((ref16 - ref).abs().max())
    err = float((got - ref).abs().max())
    band = max(1.5 * noise, 3e-2 * float(ref.abs().max())) + 1e-2
    assert err <= band, f"max|gpu - oracle| = {err:.4f}, bf16 oracle vs fp32 oracle = {noise:.4f}, band {band:.4f}"


# ---------------------------------------------------------------------------
# config 0: Qwen3-0.6B, batch 1, prefill 128 tokens then 32 greedy steps
# ---------------------------------------------------------------------------
QWEN3_06B = dict(model_type="qwen3", vocab_size=151936, hidden_size=1024, intermediate_size=3072,
                 num_hidden_layers=28, num_attention_heads=16, num_key_value_heads=8, head_dim=128,
                 max_position_embeddings=40960, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)


def _qwen06b(seed: int):
    """The 28-layer Qwen3-0.6B architecture in bf16 on the GPU, weights N(0, 0.02) drawn on the GPU
    from `seed`, norms 1."""
    from qwen_triton import QwenTritonConfig, QwenTritonForCausalLM

    cfg = QwenTritonConfig.from_hf_config(dict(QWEN3_06B))
    model = QwenTritonForCausalLM(cfg, init_weights=False).to(DEV, torch.bfloat16).eval()
    gen = torch.Generator(device=DEV).manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, 0.02, generator=gen)
    return model, cfg


def test_model_config0_full_size_prefill_and_greedy_decode():
    """Config 0 end to end: prefill 128 seed-0 ids, 32 greedy steps replayed from one captured HIP
    graph (tokens equal the eager loop's), and the logits of all 160 positions -- 128 from the
    prefill, 32 from cached decode steps -- against the fp32 CPU oracle, teacher-forced on the
    generated sequence, in the band the oracle's own bf16 run calibrates."""
    from oracle.model import ModelSpec, OracleQwen

    model, cfg = _qwen06b(0)
    V = cfg.vocab_size
    ids = torch.randint(0, V, (1, 128), generator=torch.Generator().manual_seed(0)).to(DEV)
    with torch.no_grad():
        gen_graph = model.greedy_generate(ids, max_new_tokens=32, use_graph=True)
        gen_eager = model.greedy_generate(ids, max_new_tokens=32)
    assert gen_graph.shape == (1, 160)
    assert torch.equal(gen_graph, gen_eager), "graph-replayed greedy tokens differ from the eager loop's"
    seq = gen_graph
    cd = native_calls("qh_flash_decode_prepare")
    with torch.no_grad():
        cache = model.new_cache(1, 160, torch.bfloat16, DEV)
        parts = [model(input_ids=seq[:, :128], past_key_values=cache, use_cache=True).logits.float().cpu()]
        for t in range(128, 160):
            step = model(input_ids=seq[:, t:t + 1], past_key_values=cache, use_cache=True, logits_to_keep=1)
            parts.append(step.logits.float().cpu())
    assert native_calls("qh_flash_decode_prepare") >= cd + 32 * cfg.num_hidden_layers
    got = torch.cat(parts, dim=1)[0]  # [160, V]
    params = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    spec = ModelSpec.from_config(cfg)
    ref = OracleQwen(spec, params, dtype=torch.float32).forward(seq.cpu())[0]
    ref16 = OracleQwen(spec, params, dtype=torch.bfloat16).forward(seq.cpu())[0].float()
    noise = float((ref16 - ref).abs().max())
    err = float((got - ref).abs().max())
    band = max(1.5 * noise, 3e-2 * float(ref.abs().max())) + 1e-2
    assert err <= band, f"max|gpu - oracle| = {err:.4f}, bf16 oracle vs fp32 oracle = {noise:.4f}, band {band:.4f}"
    # each greedy pick is the oracle's best token up to the band (near-ties may resolve either way)
    for t in range(128, 160):
        row = ref[t - 1]
        assert float(row[seq[0, t]]) >= float(row.max()) - band, f"step {t - 128}: token far from the oracle's argmax"
    print(f"config0: max|d| {err:.4f} (bf16 oracle noise {noise:.4f}, band {band:.4f})")


# ---------------------------------------------------------------------------
# config 4: attention at 30B-A3B shape (32 q-heads / 4 kv-heads, GQA group 8), B4 x S4096, causal
# ---------------------------------------------------------------------------
def test_flash_attention_config4_full_size():
    B, Hq, Hkv, S, D = 4, 32, 4, 4096, 128
    G = Hq // Hkv
    scale = D ** -0.5
    q, k, v, do = _randn((B, Hq, S, D), 51), _randn((B, Hkv, S, D), 52), _randn((B, Hkv, S, D), 53), \
        _randn((B, Hq, S, D), 54)
    cf, cb = native_calls("qh_flash_fwd"), native_calls("qh_flash_bwd")
    o, lse = FA.flash_forward(q, k, v, scale, True, G)
    dq, dk, dv = FA.flash_backward(q, k, v, o, do, lse, scale, True, G)
    assert native_calls("qh_flash_fwd") == cf + 1 and native_calls("qh_flash_bwd") == cb + 1
    visible = torch.ones(S, S, dtype=torch.bool, device=DEV).tril()
    worst = {"o": 0.0, "lse": 0.0, "dq": 0.0, "dk": 0.0, "dv": 0.0}
    for b in range(B):
        for hk in range(Hkv):
            dk_ref = torch.zeros(S, D, device=DEV)
            dv_ref = torch.zeros(S, D, device=DEV)
            kf, vf = k[b, hk].float(), v[b, hk].float()
            for h in range(hk * G, (hk + 1) * G):
                qf, dof = q[b, h].float(), do[b, h].float()
                s = (qf @ kf.t().contiguous()) * scale
                s.masked_fill_(~visible, float("-inf"))
                lse_ref = torch.logsumexp(s, dim=-1)
                p = torch.exp(s - lse_ref[:, None])
                o_ref = p @ vf
                ds = p * ((dof @ vf.t().contiguous()) - (dof * o_ref).sum(-1, keepdim=True))
                dq_ref = (ds @ kf) * scale
                worst["o"] = max(worst["o"], _rel_err(o[b, h], o_ref))
                worst["lse"] = max(worst["lse"], float((lse[b, h] - lse_ref).abs().max()))
                worst["dq"] = max(worst["dq"], _rel_err(dq[b, h], dq_ref))
                for key, a, r in (("o_rms", o[b, h], o_ref), ("dq_rms", dq[b, h], dq_ref)):
                    worst[key] = max(worst.get(key, 0.0), _rms_err(a, r))
                dk_ref += (ds.t().contiguous() @ qf) * scale
                dv_ref += p.t().contiguous() @ dof
            worst["dk"] = max(worst["dk"], _rel_err(dk[b, hk], dk_ref))
            worst["dv"] = max(worst["dv"], _rel_err(dv[b, hk], dv_ref))
            for key, a, r in (("dk_rms", dk[b, hk], dk_ref), ("dv_rms", dv[b, hk], dv_ref)):
                worst[key] = max(worst.get(key, 0.0), _rms_err(a, r))
    print("[fullsize] config4 attention:", worst, flush=True)
    assert worst["o"] <= 2e-2 and worst["dq"] <= 2e-2 and worst["dk"] <= 2e-2 and worst["dv"] <= 2e-2, worst
    assert max(worst[k] for k in ("o_rms", "dq_rms", "dk_rms", "dv_rms")) <= 6e-3, worst
    assert worst["lse"] <= 1e-3, worst


def test_moe_decoder_layer_config4_full_size():
    """One Qwen3-MoE decoder layer at 30B-A3B shape (hidden 2048, 32/4 heads, 128 experts, top-8,
    expert intermediate 768) on 4 x 4096 tokens, forward + backward, against an fp32 torch
    composition of the same layer (RMSNorm, q/k/v, q/k norm, RoPE, causal GQA attention, o_proj,
    residual, RMSNorm, router softmax + top-8 + renormalisation, per-expert SwiGLU, weighted
    combine, residual) under autograd. The fp32 composition takes the layer's expert choice, so that
    near-tied routings cannot flip between the two evaluations."""
    from qwen_triton import QwenTritonConfig
    from qwen_triton.models.core import QwenDecoderLayer
    from qwen_triton.modules.rotary import QwenRotaryEmbedding

    B, S, H, E, K, I, Hq, Hkv, D = 4, 4096, 2048, 128, 8, 768, 32, 4, 128
    T = B * S
    cfg = QwenTritonConfig.from_hf_config(dict(
        model_type="qwen3_moe", vocab_size=151936, hidden_size=H, intermediate_size=6144, num_hidden_layers=1,
        num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=D, moe_intermediate_size=I, num_experts=E,
        num_experts_per_tok=K, norm_topk_prob=True, decoder_sparse_step=1, mlp_only_layers=[]))
    layer = QwenDecoderLayer(cfg, 0).to(DEV, torch.bfloat16)
    gen = torch.Generator(device=DEV).manual_seed(61)
    with torch.no_grad():
        for n, p in layer.named_parameters():
            if "norm" in n:
                p.uniform_(0.8, 1.2, generator=gen)
            else:
                p.normal_(0.0, 0.02, generator=gen)
    blk = layer.mlp
    chosen = {}
    route = blk.route

    def recording_route(logits, dtype):
        w, sel = route(logits, dtype)
        chosen["sel"] = sel
        return w, sel

    blk.route = recording_route
    rot = QwenRotaryEmbedding(cfg).to(DEV)
    pos = torch.arange(S, device=DEV)[None].expand(B, S)
    x = _randn((B, S, H), 62).requires_grad_(True)
    gy = _randn((B, S, H), 63)
    cos, sin = rot(x, pos)
    cf, cu = native_calls("qh_flash_bwd"), native_calls("qh_moe_up")
    y, _ = layer(x, (cos, sin))
    y.backward(gy)
    assert native_calls("qh_flash_bwd") == cf + 1 and native_calls("qh_moe_up") == cu + 1

    # fp32 composition with autograd
    P = {n: p.detach().float().requires_grad_(True) for n, p in layer.named_parameters()}
    xf = x.detach().float().requires_grad_(True)
    cf32, sf32 = cos.float(), sin.float()
    eps = cfg.rms_norm_eps

    def rms(t, w):
        return t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + eps) * w

    def rope(t):
        half = D // 2
        return t * cf32[:, None] + torch.cat((-t[..., half:], t[..., :half]), dim=-1) * sf32[:, None]

    a = "self_attn."
    h = rms(xf, P["input_layernorm.weight"])
    q = rms((h @ P[a + "q_proj.weight"].T).view(B, S, Hq, D), P[a + "q_norm.weight"]).transpose(1, 2)
    k = rms((h @ P[a + "k_proj.weight"].T).view(B, S, Hkv, D), P[a + "k_norm.weight"]).transpose(1, 2)
    v = (h @ P[a + "v_proj.weight"].T).view(B, S, Hkv, D).transpose(1, 2)
    q, k = rope(q), rope(k)
    att = torch.nn.functional.scaled_dot_product_attention(
        q, k.repeat_interleave(Hq // Hkv, 1), v.repeat_interleave(Hq // Hkv, 1), is_causal=True, scale=D ** -0.5)
    x1 = xf + att.transpose(1, 2).reshape(B, S, Hq * D) @ P[a + "o_proj.weight"].T
    h2 = rms(x1, P["post_attention_layernorm.weight"]).view(T, H)
    probs = torch.softmax(h2 @ P["mlp.gate.weight"].T, dim=-1)
    sel = chosen["sel"]
    w = probs.gather(1, sel)
    w = w / w.sum(-1, keepdim=True)
    moe = torch.zeros_like(h2)
    for e in range(E):
        tok, slot = torch.where(sel == e)
        if tok.numel() == 0:
            continue
        pre = f"mlp.experts.{e}."
        xe = h2[tok]
        he = (torch.nn.functional.silu(xe @ P[pre + "gate_proj.weight"].T) * (xe @ P[pre + "up_proj.weight"].T))
        moe = moe.index_add(0, tok, (he @ P[pre + "down_proj.weight"].T) * w[tok, slot, None])
    yf = x1 + moe.view(B, S, H)
    yf.backward(gy.float())

    report = {"y": _rel_err(y, yf), "dx": _rel_err(x.grad, xf.grad)}
    grads = dict(layer.named_parameters())
    groups = {"attention weights": [n for n in P if n.startswith(a) and "norm" not in n],
              "norm weights": [n for n in P if "norm" in n], "router": ["mlp.gate.weight"],
              "experts": [n for n in P if "experts" in n]}
    for gname, names in groups.items():
        report[gname] = max(_rel_err(grads[n].grad, P[n].grad) for n in names)
    print("config4 layer:", {k2: f"{v2:.3e}" for k2, v2 in report.items()})
    assert report["y"] <= 2e-2 and report["dx"] <= 3e-2, report
    assert report["attention weights"] <= 4e-2 and report["router"] <= 4e-2 and report["experts"] <= 4e-2, report
    assert report["norm weights"] <= 5e-2, report


# ---------------------------------------------------------------------------
# config 2: the fused LM head + cross-entropy at 16384 tokens x 151936 classes
# ---------------------------------------------------------------------------
def test_fused_lm_head_cross_entropy_config2_full_size():
    """Loss, dX and dW of fused_linear_cross_entropy at config 2's LM-head shape against fp32 torch
    (logits in fp32 from the same bf16 inputs) and against the unfused HIP path; four blocks of 4096
    rows, each block's logits computed once, dW accumulated over the blocks in order."""
    T, H, V = 16384, 1024, 151936
    x0 = _randn((T, H), 71)
    w0 = _randn((V, H), 72, scale=0.02)
    t = torch.randint(0, V, (T,), generator=torch.Generator().manual_seed(73)).to(DEV)
    x, w = x0.clone().requires_grad_(True), w0.clone().requires_grad_(True)
    loss = K.fused_linear_cross_entropy(x, w, t)
    loss.backward()
    # fp32 reference
    xf, wf = x0.float().requires_grad_(True), w0.float().requires_grad_(True)
    lf = torch.nn.functional.cross_entropy(xf @ wf.t().contiguous(), t)
    lf.backward()
    assert abs(float(loss) - float(lf)) <= 2e-3 * abs(float(lf)), (float(loss), float(lf))
    _check(x.grad, xf.grad, 3e-2, "dX vs fp32", rms_tol=5e-3)
    _check(w.grad, wf.grad, 3e-2, "dW vs fp32", rms_tol=5e-3)
    del xf, wf, lf
    torch.cuda.empty_cache()
    # unfused HIP path (logits materialised)
    xu, wu = x0.clone().requires_grad_(True), w0.clone().requires_grad_(True)
    lu = K.triton_cross_entropy(K.triton_matmul(xu, wu), t)
    lu.backward()
    assert abs(float(loss) - float(lu)) <= 1e-5 * abs(float(lu))
    _check(x.grad, xu.grad, 1e-2, "dX vs unfused", rms_tol=1e-3)
    _check(w.grad, wu.grad, 1e-2, "dW vs unfused", rms_tol=1e-3)
