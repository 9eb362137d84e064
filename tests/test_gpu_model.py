"""Model-level GPU parity: QwenTritonForCausalLM / QwenSparseMoeBlock on the HIP
stack (bf16) against the CPU oracle (fp32, HF semantics) on the same weights.

Logits are compared teacher-forced (random-weight greedy tokens can diverge
legitimately); the band is relative to the logit scale, in the spirit of the
reference's bf16 max|dlogit| ~ 1.1 on real weights (README.md:19).
"""
from __future__ import annotations

import pytest
import torch

from oracle import ops as O
from oracle.model import ModelSpec, OracleQwen
from qwen_triton import QwenTritonConfig, QwenTritonForCausalLM, _native
from qwen_triton.modules import QwenSparseMoeBlock

pytestmark = pytest.mark.gpu


def _cfg(**kw):
    base = dict(model_type="qwen3", vocab_size=1024, hidden_size=256, intermediate_size=768, num_hidden_layers=3,
                num_attention_heads=8, num_key_value_heads=4, head_dim=64, max_position_embeddings=512,
                rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
    base.update(kw)
    return QwenTritonConfig.from_hf_config(base)


def _model(cfg, seed=0):
    torch.manual_seed(seed)
    m = QwenTritonForCausalLM.from_config(cfg)
    with torch.no_grad():
        for n, p in m.named_parameters():
            if n.endswith("norm.weight"):
                p.uniform_(0.8, 1.2)
    return m.to("cuda", torch.bfloat16).eval()


def _band(actual, ref):
    err = (actual.float().cpu() - ref.float()).abs().max().item()
    scale = ref.abs().max().item()
    assert err <= 0.03 * scale + 1e-2, f"max|d|={err} vs max|ref|={scale}"


def test_prefill_logits_match_oracle():
    cfg = _cfg()
    m = _model(cfg)
    ids = torch.randint(0, cfg.vocab_size, (2, 77), generator=torch.Generator().manual_seed(1))
    c0 = _native.CALLS["qh_flash_fwd"]
    with torch.no_grad():
        out = m(input_ids=ids.cuda(), use_cache=False).logits
    assert _native.CALLS["qh_flash_fwd"] == c0 + cfg.num_hidden_layers  # causal prefill runs flash attention
    ref = OracleQwen(ModelSpec.from_config(cfg), m.state_dict()).forward(ids)
    _band(out, ref)


@pytest.mark.parametrize("window", [None, 40])
def test_padding_and_window_masks_in_the_flash_kernel(monkeypatch, window):
    """Left-padded prefill and a cached decode step (and a sliding window on the upper layers) take
    the masked flash kernel; their logits on the real tokens agree with the same model applying the
    reference's additive mask through fp32 SDPA."""
    from qwen_triton.modules.attention import CausalPaddingMask

    kw = dict(use_sliding_window=True, sliding_window=window, max_window_layers=1) if window else {}
    cfg = _cfg(**kw)
    m = _model(cfg)
    gen = torch.Generator().manual_seed(2)
    ids = torch.randint(0, cfg.vocab_size, (3, 90), generator=gen).cuda()
    mask = torch.ones_like(ids)
    mask[1, :70] = 0
    mask[2, :13] = 0
    nxt = torch.randint(0, cfg.vocab_size, (3, 1), generator=gen).cuda()

    def run(am):
        with torch.no_grad():
            p = m(input_ids=ids, attention_mask=am, use_cache=True)
            d = m(input_ids=nxt, attention_mask=torch.cat((am, torch.ones_like(nxt)), 1),
                  past_key_values=p.past_key_values, use_cache=True)
        return p.logits.float().cpu(), d.logits.float().cpu()

    c0 = _native.CALLS["qh_flash_fwd_masked"]
    got = run(mask)
    assert _native.CALLS["qh_flash_fwd_masked"] == c0 + 2 * cfg.num_hidden_layers
    unpadded = run(torch.ones_like(mask))  # what ignoring the padding would give
    monkeypatch.setattr(CausalPaddingMask, "kernel_args", lambda self, q, k: None)
    exp = run(mask)
    padded = mask.bool().cpu()
    padded[0] = False  # the real tokens of the padded sequences
    for g, e, u, rows in zip(got, exp, unpadded, (padded, torch.tensor([[False], [True], [True]]))):
        _band(g[rows], e[rows])
        # the padding is live: ignoring it moves these logits far more than the kernel's error
        assert (g[rows] - e[rows]).abs().max() < 0.2 * (u[rows] - e[rows]).abs().max()


def test_cached_decode_matches_full_forward_and_oracle():
    cfg = _cfg()
    m = _model(cfg, seed=1)
    ids = torch.randint(0, cfg.vocab_size, (3, 40), generator=torch.Generator().manual_seed(2)).cuda()
    with torch.no_grad():
        p = m(input_ids=ids[:, :33], use_cache=True)
        steps = []
        cache = p.past_key_values
        for t in range(33, 40):
            o = m(input_ids=ids[:, t:t + 1], past_key_values=cache, use_cache=True, logits_to_keep=1)
            steps.append(o.logits)
        full = m(input_ids=ids, use_cache=False).logits
    dec = torch.cat(steps, dim=1)
    _band(dec, full[:, 33:].float().cpu())
    ref = OracleQwen(ModelSpec.from_config(cfg), m.state_dict()).forward(ids.cpu())
    _band(dec, ref[:, 33:])


def test_chunked_prefill_on_cache_uses_bottom_right_causal():
    cfg = _cfg()
    m = _model(cfg, seed=2)
    ids = torch.randint(0, cfg.vocab_size, (1, 50), generator=torch.Generator().manual_seed(3)).cuda()
    with torch.no_grad():
        p = m(input_ids=ids[:, :30], use_cache=True)
        chunk = m(input_ids=ids[:, 30:], past_key_values=p.past_key_values, use_cache=True).logits
        full = m(input_ids=ids, use_cache=False).logits
    _band(chunk, full[:, 30:].float().cpu())


def test_greedy_generate_teacher_forced():
    cfg = _cfg()
    m = _model(cfg, seed=3)
    ids = torch.randint(0, cfg.vocab_size, (1, 16), generator=torch.Generator().manual_seed(4)).cuda()
    gen = m.greedy_generate(ids, max_new_tokens=8)
    assert gen.shape == (1, 24)
    with torch.no_grad():
        logits = m(input_ids=gen, use_cache=False).logits
    ref = OracleQwen(ModelSpec.from_config(cfg), m.state_dict()).forward(gen.cpu())
    _band(logits, ref)


def test_training_step_loss_and_grads():
    cfg = _cfg(num_hidden_layers=2)
    m = _model(cfg, seed=4).train()
    ids = torch.randint(0, cfg.vocab_size, (2, 64), generator=torch.Generator().manual_seed(5)).cuda()
    out = m(input_ids=ids, labels=ids)
    ref_logits = OracleQwen(ModelSpec.from_config(cfg), m.state_dict()).forward(ids.cpu())
    ref_loss = O.cross_entropy(ref_logits[:, :-1].reshape(-1, cfg.vocab_size), ids[:, 1:].reshape(-1).cpu())[0]
    assert abs(out.loss.item() - ref_loss.item()) < 2e-2 * max(1.0, ref_loss.item())
    c0 = _native.CALLS["qh_flash_bwd"]
    out.loss.backward()
    assert _native.CALLS["qh_flash_bwd"] == c0 + cfg.num_hidden_layers
    for n, p in m.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), n


def _grad_agreement(got: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    """(max|got - ref| / max|ref|, cosine similarity) of a gradient against its oracle."""
    g, r = got.detach().double().cpu().flatten(), ref.detach().double().cpu().flatten()
    rel = float((g - r).abs().max()) / max(float(r.abs().max()), 1e-30)
    cos = float(g @ r) / max(float(g.norm() * r.norm()), 1e-300)
    return rel, cos


def test_training_gradients_match_oracle_autograd():
    """Every parameter gradient of a bf16 training step (embedding, norms, q/k/v/o, MLP, tied LM
    head; flash-attention, RMSNorm, RoPE, SiLU-mul, CE and GEMM backward kernels) against autograd
    through the fp64 CPU oracle on the same (bf16-rounded) weights."""
    import torch.nn.functional as F

    cfg = _cfg(num_hidden_layers=2)
    m = _model(cfg, seed=6).train()
    ids = torch.randint(0, cfg.vocab_size, (2, 64), generator=torch.Generator().manual_seed(7)).cuda()
    out = m(input_ids=ids, labels=ids)
    out.loss.backward()
    orc = OracleQwen(ModelSpec.from_config(cfg), m.state_dict(), dtype=torch.float64)
    for k in list(orc.p):
        if k != "lm_head.weight":
            orc.p[k] = orc.p[k].clone().requires_grad_(True)
    orc.p["lm_head.weight"] = orc.p["model.embed_tokens.weight"]  # tied
    logits = orc.forward(ids.cpu())
    loss = F.cross_entropy(logits[:, :-1].reshape(-1, cfg.vocab_size), ids[:, 1:].reshape(-1).cpu())
    loss.backward()
    assert abs(out.loss.item() - loss.item()) <= 1e-2 * loss.item()
    worst = []
    for n, p in m.named_parameters():
        rel, cos = _grad_agreement(p.grad, orc.p[n].grad)
        worst.append((rel, cos, n))
        assert cos >= 0.999 and rel <= 0.05, f"{n}: max rel {rel:.3e}, cosine {cos:.6f}"
    print("worst gradient agreement:", max(worst)[:2], min(worst, key=lambda t: t[1])[1:])


def test_moe_block_gradients_match_oracle_autograd():
    """QwenSparseMoeBlock training (grouped expert kernels + router softmax/top-k backward + gate GEMM
    backward) against fp64 autograd through the oracle (E=8, top-2, 300 tokens): output, input
    gradient, router weight gradient and every expert weight gradient. The oracle takes the GPU's
    expert choice (checked equal to top-k on the GPU probabilities by the forward test) so that
    near-tied routings cannot flip between the two evaluations."""
    E, K, H, I, T = 8, 2, 256, 128, 300
    cfg = QwenTritonConfig.from_hf_config(dict(
        model_type="qwen3_moe", vocab_size=64, hidden_size=H, intermediate_size=512, num_hidden_layers=1,
        num_attention_heads=4, num_key_value_heads=2, head_dim=64, moe_intermediate_size=I, num_experts=E,
        num_experts_per_tok=K, norm_topk_prob=True, decoder_sparse_step=1, mlp_only_layers=[]))
    torch.manual_seed(1)
    blk = QwenSparseMoeBlock(cfg)
    with torch.no_grad():
        for p in blk.parameters():
            p.normal_(0.0, 0.05)
    blk = blk.to("cuda", torch.bfloat16).train()
    x = torch.randn(1, T, H, generator=torch.Generator().manual_seed(8)).to("cuda", torch.bfloat16)
    x.requires_grad_(True)
    gout = torch.randn(1, T, H, generator=torch.Generator().manual_seed(9)).to("cuda", torch.bfloat16)
    chosen = {}
    route = blk.route

    def recording_route(logits, dtype):
        w, sel = route(logits, dtype)
        chosen["sel"] = sel
        return w, sel

    blk.route = recording_route
    c0 = _native.CALLS["qh_moe_up"]
    out, _ = blk(x)
    out.backward(gout)
    assert _native.CALLS["qh_moe_up"] == c0 + 1  # the grouped training kernels ran
    wg = torch.stack([ex.gate_proj.weight for ex in blk.experts])
    wu = torch.stack([ex.up_proj.weight for ex in blk.experts])
    wd = torch.stack([ex.down_proj.weight for ex in blk.experts])
    ref, dx, dgw, dwg, dwu, dwd = O.moe_block_grads(x.view(T, H), blk.gate.weight, wg, wu, wd, K, gout.view(T, H),
                                                    True, experts=chosen["sel"].cpu())
    checks = [("out", out.view(T, H), ref), ("dx", x.grad.view(T, H), dx), ("d gate", blk.gate.weight.grad, dgw),
              ("d gate_proj", torch.stack([ex.gate_proj.weight.grad for ex in blk.experts]), dwg),
              ("d up_proj", torch.stack([ex.up_proj.weight.grad for ex in blk.experts]), dwu),
              ("d down_proj", torch.stack([ex.down_proj.weight.grad for ex in blk.experts]), dwd)]
    for what, got, exp in checks:
        rel, cos = _grad_agreement(got, exp)
        print(f"{what}: max rel {rel:.3e}, cosine {cos:.6f}")
        assert cos >= 0.999 and rel <= 0.04, f"{what}: max rel {rel:.3e}, cosine {cos:.6f}"


def test_loader_checkpoint_on_gpu_matches_golden_logits(tmp_path):
    """A safetensors checkpoint of the golden HF weights (fused experts, wrapper prefix) loaded by
    from_pretrained_hf straight to the GPU in bf16: logits within the bf16 band of HF's."""
    from test_loader_cpu import golden, write_checkpoint

    for name, layout in (("qwen3_tiny.npz", dict(prefix="model.language_model.")), ("qwen3_moe_tiny.npz", {})):
        params, ids, logits, raw = golden(name)
        write_checkpoint(tmp_path / name, params, raw, **layout)
        model = QwenTritonForCausalLM.from_pretrained_hf(str(tmp_path / name), device="cuda", dtype=torch.bfloat16)
        assert next(model.parameters()).is_cuda
        with torch.no_grad():
            ours = model(input_ids=ids.cuda(), use_cache=False).logits
        _band(ours, logits)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rotary_table_rows_equal_the_per_call_computation(dtype):
    """The cached cos/sin table (one gather per forward) gives the same bits as computing cos/sin of
    the positions directly, at positions up to 40959 and for a batch of position rows."""
    from qwen_triton.modules.rotary import QwenRotaryEmbedding

    rot = QwenRotaryEmbedding(_cfg(max_position_embeddings=40960)).to("cuda")
    x = torch.zeros(1, 1, 8, device="cuda", dtype=dtype)
    pos = torch.cat((torch.arange(0, 300), torch.tensor([2047, 2048, 4095, 40959]))).cuda()[None]
    c0, s0 = rot(x, pos)
    c1, s1 = rot(x, pos, max_position=40959)
    assert torch.equal(c0, c1) and torch.equal(s0, s1)
    pos2 = torch.randint(0, 5000, (3, 17), generator=torch.Generator().manual_seed(11)).cuda()
    c0, s0 = rot(x, pos2)
    c1, s1 = rot(x, pos2, max_position=4999)
    assert torch.equal(c0, c1) and torch.equal(s0, s1)
    assert c1.stride() == s1.stride() and c1.stride(-1) == 1


def test_moe_block_routing_exact_and_output_close():
    cfg = QwenTritonConfig.from_hf_config(dict(
        model_type="qwen3_moe", vocab_size=64, hidden_size=256, intermediate_size=512, num_hidden_layers=1,
        num_attention_heads=4, num_key_value_heads=2, head_dim=64, moe_intermediate_size=128, num_experts=16,
        num_experts_per_tok=4, norm_topk_prob=True, decoder_sparse_step=1, mlp_only_layers=[]))
    torch.manual_seed(0)
    blk = QwenSparseMoeBlock(cfg)
    with torch.no_grad():
        for p in blk.parameters():
            p.normal_(0.0, 0.05)
    blk = blk.to("cuda", torch.bfloat16)
    x = torch.randn(2, 40, 256, generator=torch.Generator().manual_seed(6)).to("cuda", torch.bfloat16)
    with torch.no_grad():
        out, logits = blk(x)
        w, e = blk.route(logits, torch.bfloat16)
    from qwen_triton.kernels import triton_softmax

    probs = triton_softmax(logits.float())
    assert torch.equal(e.cpu(), O.topk(probs, 4)[1])  # top-k bit-exact on the op's own input
    torch.testing.assert_close(probs.cpu().double(), O.softmax(logits.float()), atol=1e-6, rtol=1e-5)
    wg = torch.stack([ex.gate_proj.weight for ex in blk.experts]).float().cpu()
    wu = torch.stack([ex.up_proj.weight for ex in blk.experts]).float().cpu()
    wd = torch.stack([ex.down_proj.weight for ex in blk.experts]).float().cpu()
    ref, *_ = O.moe_block(x.view(-1, 256), None, wg, wu, wd, 4, True, router_logits=logits)
    _band(out.view(-1, 256), ref)


def test_decode_step_graph_replays_match_eager():
    cfg = _cfg()
    m = _model(cfg, seed=5)
    B, ctx = 4, 100
    cache = m.new_cache(B, ctx + 8, torch.bfloat16, "cuda")
    gen = torch.Generator(device="cuda").manual_seed(0)
    for i in range(cfg.num_hidden_layers):
        cache.key_cache[i][:, :, :ctx].normal_(generator=gen)
        cache.value_cache[i][:, :, :ctx].normal_(generator=gen)
    ids = torch.randint(0, cfg.vocab_size, (B, 1), device="cuda", generator=gen)

    def step():
        cache.attention_lengths = [ctx] * cfg.num_hidden_layers
        return m(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=1).logits

    with torch.no_grad():
        eager = step().clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = step()
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
            step()  # eager work between replays
            torch.cuda.synchronize()


@pytest.mark.parametrize("seq,per_batch_pos", [(1, False), (5, False), (5, True)])
def test_fused_attention_prepare_matches_unfused_path(seq, per_batch_pos):
    # inference takes one fused q/k-norm + RoPE + cache-write launch; it must equal the
    # separate kernels (autograd path) bit for bit, in the output and in both caches
    from qwen_triton.modules.cache import QwenTritonCache

    cfg = _cfg()
    m = _model(cfg, seed=6)
    attn = m.model.layers[1].self_attn
    B, ctx = 3, 9
    gen = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn(B, seq, cfg.hidden_size, device="cuda", dtype=torch.bfloat16, generator=gen)
    pos = torch.arange(ctx, ctx + seq, device="cuda")
    pid = (pos[None] + torch.arange(B, device="cuda")[:, None]) if per_batch_pos else pos[None]
    cos, sin = m.model.rotary_emb(x, pid)
    caches = []
    for _ in range(2):
        c = QwenTritonCache(cfg.num_hidden_layers, cfg.layer_types)
        c.reserve(1, B, cfg.num_key_value_heads, 32, cfg.head_dim, torch.bfloat16, "cuda")
        g2 = torch.Generator(device="cuda").manual_seed(8)
        c.key_cache[1][:, :, :ctx].normal_(generator=g2)
        c.value_cache[1][:, :, :ctx].normal_(generator=g2)
        c.attention_lengths[1] = ctx
        caches.append(c)
    c0 = _native.CALLS["qh_attn_prepare"]
    with torch.enable_grad():
        ref = attn(x, (cos, sin), None, caches[0], pos, max_position=ctx + seq - 1).detach()
    assert _native.CALLS["qh_attn_prepare"] == c0
    with torch.no_grad():
        out = attn(x, (cos, sin), None, caches[1], pos, max_position=ctx + seq - 1)
    assert _native.CALLS["qh_attn_prepare"] == c0 + 1
    assert caches[0].attention_lengths[1] == caches[1].attention_lengths[1] == ctx + seq
    n = ctx + seq  # rows past the valid length are uninitialised storage
    assert torch.equal(caches[0].key_cache[1][:, :, :n], caches[1].key_cache[1][:, :, :n])
    assert torch.equal(caches[0].value_cache[1][:, :, :n], caches[1].value_cache[1][:, :, :n])
    assert torch.equal(ref, out)


def test_inference_fusions_match_autograd_path_bitwise(monkeypatch):
    # no_grad enables the fused inference kernels (grouped GEMMs, attention prep,
    # add+norm chains); each is built to equal its unfused chain exactly, so the
    # whole model must give identical logits in both modes, prefill and decode.
    # The norm-in-GEMM layer path sums squares in another order (checked
    # separately below), so it is switched off here.
    from qwen_triton.models import core

    monkeypatch.setattr(core, "FUSE_NORM_GEMM", False)
    cfg = _cfg()
    m = _model(cfg, seed=9)
    # frozen weights: with grad mode on nothing requires grad, so kernel choices
    # (e.g. the split-KV decode kernel for one query) are those of no_grad and
    # only the fusions differ between the two runs
    for p in m.parameters():
        p.requires_grad_(False)
    ids = torch.randint(0, cfg.vocab_size, (2, 70), generator=torch.Generator().manual_seed(10)).cuda()
    outs = {}
    for mode in ("fused", "plain"):
        ctx = torch.no_grad() if mode == "fused" else torch.enable_grad()
        with ctx:
            p = m(input_ids=ids[:, :66], use_cache=True)
            steps = [p.logits.detach()]
            cache = p.past_key_values
            for t in range(66, 70):
                o = m(input_ids=ids[:, t:t + 1], past_key_values=cache, use_cache=True)
                steps.append(o.logits.detach())
        outs[mode] = steps
    for a, b in zip(outs["fused"], outs["plain"]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("batch", [1, 3])
def test_fused_layer_path_matches_separate_kernels(monkeypatch, batch):
    # Decode steps through QwenDecoderLayer.forward_fused (norms inside the q/k/v and gate/up
    # products, residual adds inside o_proj and down_proj: five launches per layer) against the
    # same steps on the separate kernels, and both against the fp32 CPU oracle teacher-forced.
    from qwen_triton.models import core

    cfg = _cfg()
    m = _model(cfg, seed=21)
    ids = torch.randint(0, cfg.vocab_size, (batch, 40), generator=torch.Generator().manual_seed(22)).cuda()
    outs = {}
    for fused in (True, False):
        monkeypatch.setattr(core, "FUSE_NORM_GEMM", fused)
        c0 = _native.CALLS["qh_gemm_multi_ex"] + _native.CALLS["qh_gemm_multi_rms"]
        with torch.no_grad():
            p = m(input_ids=ids[:, :33], use_cache=True)
            steps = [p.logits[:, -1]]
            cache = p.past_key_values
            for t in range(33, 40):
                steps.append(m(input_ids=ids[:, t:t + 1], past_key_values=cache, use_cache=True).logits[:, -1])
        launched = _native.CALLS["qh_gemm_multi_ex"] + _native.CALLS["qh_gemm_multi_rms"] - c0
        # fused launches per layer and token (q/k/v, o_proj, gate/up, down: 4; the prefill of
        # 33 * batch rows takes the fused path too when it has at most 128 rows)
        per_pass = 4 * cfg.num_hidden_layers
        expect = per_pass * (7 + (1 if 33 * batch <= 128 else 0)) if fused else 0
        assert launched == expect
        outs[fused] = torch.stack(steps, 1).float().cpu()
    a, b = outs[True], outs[False]
    # one rounding step of a normalised element moves a logit by far less than the bf16 band
    err = (a - b).abs().max().item()
    assert err <= 0.01 * b.abs().max().item() + 1e-2, err
    ref = OracleQwen(ModelSpec.from_config(cfg), m.state_dict(), dtype=torch.float32).forward(ids.cpu())
    _band(a, ref[:, 32:40])
    # reruns are bitwise equal
    monkeypatch.setattr(core, "FUSE_NORM_GEMM", True)
    with torch.no_grad():
        p = m(input_ids=ids[:, :33], use_cache=True)
        again = [p.logits[:, -1]]
        for t in range(33, 40):
            again.append(m(input_ids=ids[:, t:t + 1], past_key_values=p.past_key_values, use_cache=True).logits[:, -1])
    assert torch.equal(torch.stack(again, 1).float().cpu(), a)


@pytest.mark.parametrize("moe,prompt", [(False, 19), (True, 19), (False, 300), (False, 600)])
def test_greedy_generate_graph_replay_matches_eager(moe, prompt):
    """greedy_generate(use_graph=True): one captured decode step replayed per token, with the
    position and valid lengths advanced on the device. The eager loop decodes through the same
    device state, so the tokens are identical at every cache length (caches of 43, 324 and 624
    positions, planned as one to several key splits of the decode attention); the replays (not
    Python calls) do the work."""
    extra = dict(model_type="qwen3_moe", moe_intermediate_size=128, num_experts=8, num_experts_per_tok=2,
                 norm_topk_prob=True, decoder_sparse_step=1, mlp_only_layers=[]) if moe else {}
    cfg = _cfg(max_position_embeddings=1024, **extra)
    m = _model(cfg, seed=5)
    ids = torch.randint(0, cfg.vocab_size, (2, prompt), generator=torch.Generator().manual_seed(6)).cuda()
    new = 24
    with torch.no_grad():
        eager = m.greedy_generate(ids, max_new_tokens=new)
        c0 = _native.CALLS["qh_flash_decode"]
        graph = m.greedy_generate(ids, max_new_tokens=new, use_graph=True)
        launched = _native.CALLS["qh_flash_decode"] - c0
        again = m.greedy_generate(ids, max_new_tokens=new, use_graph=True)
    assert graph.shape == (2, prompt + new)
    assert torch.equal(graph, eager)
    assert torch.equal(again, eager)
    # decode attention entered from Python twice per layer (the eager second token and the
    # capture), not once per generated token
    assert launched == 2 * cfg.num_hidden_layers


def test_graph_runner_follows_in_place_weight_updates():
    """Cached greedy graphs read the parameters and tensors derived from them (norm-folded
    weights, rotary tables) by address. After an in-place update of the weights (as a checkpoint
    load's ``copy_`` or an optimizer step does) the next graph generation must equal the eager
    loop on the new weights, not replay the old folded copies; a regrown rotary table must not
    free what an older runner reads."""
    cfg = _cfg(max_position_embeddings=1024)
    m = _model(cfg, seed=31)
    ids = torch.randint(0, cfg.vocab_size, (2, 19), generator=torch.Generator().manual_seed(32)).cuda()
    new = 12
    with torch.no_grad():
        g0 = m.greedy_generate(ids, max_new_tokens=new, use_graph=True)
        assert torch.equal(g0, m.greedy_generate(ids, max_new_tokens=new))
        donor = _model(cfg, seed=33)
        for p, q in zip(m.parameters(), donor.parameters()):
            p.copy_(q)  # in place: same storage, new values
        eager = m.greedy_generate(ids, max_new_tokens=new)
        graph = m.greedy_generate(ids, max_new_tokens=new, use_graph=True)
        assert not torch.equal(eager, g0)
        assert torch.equal(graph, eager)
        # a longer generation regrows the rotary tables; the runner of the shorter one still replays
        m.greedy_generate(ids, max_new_tokens=700, use_graph=False)
        assert torch.equal(m.greedy_generate(ids, max_new_tokens=new, use_graph=True), eager)


def test_fold_switch_off_keeps_no_weight_copies(monkeypatch):
    """With ``FOLD_NORM_WEIGHTS`` off the norm-fused products scale the weight fragments in the
    launch (no folded copy is kept) and give the folded path's bits for more than 4 rows;
    ``release_folded_weights`` frees the copies the folded path made."""
    from qwen_triton.kernels import matmul

    cfg = _cfg()
    m = _model(cfg, seed=35)
    ids = torch.randint(0, cfg.vocab_size, (8, 12), generator=torch.Generator().manual_seed(36)).cuda()
    outs = {}
    for fold in (True, False):
        monkeypatch.setattr(matmul, "FOLD_NORM_WEIGHTS", fold)
        assert m.release_folded_weights() >= 0
        c0 = _native.CALLS["qh_gemm_multi_rms"]
        with torch.no_grad():
            p = m(input_ids=ids[:, :8], use_cache=True)
            steps = [p.logits[:, -1]]
            for t in range(8, 12):
                steps.append(m(input_ids=ids[:, t:t + 1], past_key_values=p.past_key_values,
                               use_cache=True).logits[:, -1])
        outs[fold] = torch.stack(steps, 1)
        kept = matmul.folded_weight_tensors(m)
        if fold:
            assert _native.CALLS["qh_gemm_multi_rms"] > c0 and kept
            qkv = sum(w.numel() for w in (m.model.layers[0].self_attn.q_proj.weight,
                                          m.model.layers[0].self_attn.k_proj.weight,
                                          m.model.layers[0].self_attn.v_proj.weight,
                                          m.model.layers[0].mlp.gate_proj.weight,
                                          m.model.layers[0].mlp.up_proj.weight))
            assert sum(w.numel() for w in kept) == qkv * cfg.num_hidden_layers
        else:
            assert _native.CALLS["qh_gemm_multi_rms"] == c0 and not kept
    assert torch.equal(outs[True], outs[False])
    monkeypatch.setattr(matmul, "FOLD_NORM_WEIGHTS", True)
    assert m.release_folded_weights() == 0


def test_fused_decode_prepare_in_model_bitwise(monkeypatch):
    # 64 sequences x 8 kv-heads: decode steps take qh_flash_decode_prepare (norm, RoPE and cache
    # writes inside the decode-attention kernel); the separate prepare pass must give identical
    # logits and caches, eager and in a captured greedy decode
    from qwen_triton.modules import attention as attn_mod

    cfg = _cfg(hidden_size=256, num_attention_heads=16, num_key_value_heads=8, head_dim=128, num_hidden_layers=2,
               vocab_size=512)
    m = _model(cfg, seed=41)
    ids = torch.randint(0, cfg.vocab_size, (64, 6), generator=torch.Generator().manual_seed(42)).cuda()
    outs = {}
    for fused in (True, False):
        monkeypatch.setattr(attn_mod, "FUSE_DECODE_PREPARE", fused)
        c0 = _native.CALLS["qh_flash_decode_prepare"]
        with torch.no_grad():
            p = m(input_ids=ids[:, :3], use_cache=True)
            steps = [p.logits[:, -1]]
            cache = p.past_key_values
            for t in range(3, 6):
                steps.append(m(input_ids=ids[:, t:t + 1], past_key_values=cache, use_cache=True).logits[:, -1])
        assert _native.CALLS["qh_flash_decode_prepare"] - c0 == (3 * cfg.num_hidden_layers if fused else 0)
        outs[fused] = (torch.stack(steps, 1), [c[:, :, :6].clone() for c in cache.key_cache])
    assert torch.equal(outs[True][0], outs[False][0])
    for a, b in zip(outs[True][1], outs[False][1]):
        assert torch.equal(a, b)
    monkeypatch.setattr(attn_mod, "FUSE_DECODE_PREPARE", True)
    with torch.no_grad():
        eager = m.greedy_generate(ids[:, :3], max_new_tokens=8)
        graph = m.greedy_generate(ids[:, :3], max_new_tokens=8, use_graph=True)
    assert torch.equal(graph, eager)


def test_config0_like_decode_takes_fused_prepare():
    # batch 1, head_dim 128, short cache: decode steps take qh_flash_decode_prepare; greedy tokens
    # equal with and without the captured graph, logits within the band of the fp32 oracle
    cfg = _cfg(hidden_size=256, num_attention_heads=16, num_key_value_heads=8, head_dim=128, num_hidden_layers=2,
               vocab_size=512)
    m = _model(cfg, seed=51)
    ids = torch.randint(0, cfg.vocab_size, (1, 20), generator=torch.Generator().manual_seed(52)).cuda()
    c0 = _native.CALLS["qh_flash_decode_prepare"]
    with torch.no_grad():
        eager = m.greedy_generate(ids, max_new_tokens=12)
        graph = m.greedy_generate(ids, max_new_tokens=12, use_graph=True)
    assert _native.CALLS["qh_flash_decode_prepare"] > c0
    assert torch.equal(graph, eager)
    with torch.no_grad():
        p = m(input_ids=eager[:, :20], use_cache=True)
        steps = [p.logits[:, -1]]
        for t in range(20, eager.shape[1] - 1):
            steps.append(m(input_ids=eager[:, t:t + 1], past_key_values=p.past_key_values, use_cache=True).logits[:, -1])
    ref = OracleQwen(ModelSpec.from_config(cfg), m.state_dict(), dtype=torch.float32).forward(eager[:, :-1].cpu())
    _band(torch.stack(steps, 1).float().cpu(), ref[:, 19:])


def test_qwen3_next_model_on_gpu_matches_golden_logits():
    """The golden Qwen3-Next model in bf16 on the GPU (linear-attention layers on the gated-delta
    kernel, gated full attention on flash attention): logits within the bf16 band of HF's, and
    token-by-token decoding through the caches within the band of the full forward."""
    from test_model_cpu import _next_model

    model, ids, logits = _next_model()
    model = model.to("cuda", torch.bfloat16)
    ids = ids.cuda()
    c0 = _native.CALLS["qh_gated_delta_rule"]
    with torch.no_grad():
        ours = model(input_ids=ids, use_cache=False).logits
        assert _native.CALLS["qh_gated_delta_rule"] == c0 + 2  # two linear-attention layers
        _band(ours, logits)
        out = model(input_ids=ids[:, :5], use_cache=True)
        cache, steps = out.past_key_values, [out.logits]
        for t in range(5, ids.shape[1]):
            o = model(input_ids=ids[:, t:t + 1], past_key_values=cache, use_cache=True)
            cache = o.past_key_values
            steps.append(o.logits)
    _band(torch.cat(steps, dim=1), logits)
