"""Throughput benchmark of the Qwen3 operator stack on one MI355X.

Default (``python bench.py``): the Qwen3-0.6B-architecture decode step of
BASELINE config 3 — 64 sequences, each with a 2048-token bf16 KV cache
(N(0,1)), one new token at position 2048 through all 28 layers — captured once
as a HIP graph and replayed ``--steps`` times. ``value`` is decode tokens/s
(64 tokens per step). The same JSON line also carries:

* config 0 on the GPU: bs1 prefill of 128 tokens and 32 greedy decode steps;
* ``roofline`` of the dominant kernel (decode attention with its row preparation,
  HBM-bound): algorithmic bytes per launch (K/V cache read, the step's q/k/v rows
  read, the output and new cache rows written) / average launch time from HIP
  events on the launch stream;
* ``cpu_baseline``: the CPU oracle (fp32 torch, HF semantics) decoding a
  bounded sample of the same workload on the host cores.

``--workload fa|dense|gemm`` time the other BASELINE configs' kernels and
``--workload roofline`` runs only the dominant kernel plus a 1 GiB calibration
copy (used for the rocprofv3 counter passes); each prints its own JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "qwen-triton_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "Qwen3-0.6B prefill/decode tok/s on 1 MI355X + % of MFMA/HBM roofline"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

# HBM bytes per launch of the decode attention as the config-3 step runs it (one
# fa_decode_wg_kernel<bf16,128,2,PREP> dispatch on the interleaved K/V cache, non-temporal loads),
# from the two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) of `bench.py --workload roofline`,
# each scaled by the same counter's reading for a 1 GiB copy (fetch x 1048576 / 524307.5, write
# x 1.000): 264342.7 KiB x 1.99993 + 512 KiB = 541,878,003 bytes (1.0069x the algorithmic bytes;
# the rest is every wave's own copy of the rows' norm weights and cos/sin).
DECODE_TRAFFIC_BYTES = 541_878_003

QWEN3_06B = dict(model_type="qwen3", vocab_size=151936, hidden_size=1024, intermediate_size=3072,
                 num_hidden_layers=28, num_attention_heads=16, num_key_value_heads=8, head_dim=128,
                 max_position_embeddings=40960, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_model(dtype, device, layers=None):
    import torch
    from qwen_triton import QwenTritonConfig, QwenTritonForCausalLM

    cfg = dict(QWEN3_06B)
    if layers is not None:
        cfg["num_hidden_layers"] = layers
    config = QwenTritonConfig.from_hf_config(cfg)
    torch.manual_seed(0)
    model = QwenTritonForCausalLM(config, init_weights=False)
    gen = torch.Generator().manual_seed(0)
    with torch.no_grad():  # N(0, 0.02) weights in parameter order, norms = 1
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
    return model.to(device=device, dtype=dtype).eval()


def sync():
    import torch

    torch.cuda.synchronize()


# ---------------------------------------------------------------------------
# config 3: decode step, batch 64, 2048-token cache
# ---------------------------------------------------------------------------
def fill_cache(model, batch, ctx, capacity, seed=0):
    import torch

    cfg = model.config
    cache = model.new_cache(batch, capacity, torch.bfloat16, "cuda")
    gen = torch.Generator(device="cuda").manual_seed(seed)
    for i in range(cfg.num_hidden_layers):
        cache.key_cache[i][:, :, :ctx].normal_(generator=gen)
        cache.value_cache[i][:, :, :ctx].normal_(generator=gen)
        cache.attention_lengths[i] = ctx
    return cache


def decode_step_fn(model, cache, ids, ctx):
    import torch
    from qwen_triton import _native

    batch, vocab = ids.shape[0], model.config.vocab_size
    nxt = torch.empty((batch,), dtype=torch.long, device=ids.device)
    ws = _native.workspace(_native.call("qh_greedy_step_workspace", batch, vocab), ids.device)

    def step():
        cache.attention_lengths = [ctx] * len(cache.attention_lengths)
        logits = model(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=1).logits
        # greedy pick as greedy_generate's captured step makes it (qh_greedy_step: torch.argmax's
        # tie and NaN rules, two launches), into a preallocated buffer: the next input ids
        last = logits[:, -1]
        _native.call("qh_greedy_step", last.data_ptr(), last.stride(0), batch, vocab, nxt.data_ptr(), None, 0, 0,
                     None, None, None, ws.data_ptr(), ws.numel(), _native.dtype_code(last.dtype),
                     _native.stream(last.device))
        return nxt

    return step


def bench_decode(model, steps, warmup, use_graph=True, batch=64, ctx=2048):
    import torch

    cache = fill_cache(model, batch, ctx, capacity=ctx + 64)
    ids = torch.randint(0, model.config.vocab_size, (batch, 1), generator=torch.Generator().manual_seed(0)).cuda()
    step = decode_step_fn(model, cache, ids, ctx)
    with torch.no_grad():
        for _ in range(max(1, warmup)):
            eager_tok = step().clone()
        sync()
        t0 = time.perf_counter()
        n_eager = max(3, min(steps, 10))
        for _ in range(n_eager):
            step()
        sync()
        eager_ms = (time.perf_counter() - t0) * 1e3 / n_eager
        log(f"decode eager: {eager_ms:.3f} ms/step")
        graph_ms = None
        if use_graph:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                step()
            torch.cuda.current_stream().wait_stream(s)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                graph_tok = step()
            for _ in range(max(1, warmup)):
                g.replay()
            sync()
            if not torch.equal(graph_tok, eager_tok):
                raise RuntimeError("graph replay disagrees with the eager decode step")
            t0 = time.perf_counter()
            for _ in range(steps):
                g.replay()
            sync()
            graph_ms = (time.perf_counter() - t0) * 1e3 / steps
            log(f"decode graph: {graph_ms:.3f} ms/step")
    return cache, eager_ms, graph_ms


def decode_layer_launch(batch=64, hq=16, hkv=8, d=128, ctx=2048, seed=0):
    """One layer's decode attention as the config-3 step runs it (qh_flash_decode_prepare: the q/k
    norm, RoPE and cache writes of the step inside the decode kernel) on synthetic inputs of that
    shape: a 2048-token bf16 cache (capacity 2112, key and value rows interleaved as the model's cache
    lays them out), the new token at position 2048. Returns
    (launch, algorithmic bytes per launch)."""
    import torch
    from qwen_triton import _native

    g = torch.Generator(device="cuda").manual_seed(seed)
    bf = torch.bfloat16
    cap, sk = ctx + 64, ctx + 1
    # the model cache's layout: key and value rows interleaved in one buffer
    kv = torch.randn(batch, hkv, cap, 2, d, device="cuda", dtype=bf, generator=g)
    kc, vc = kv[:, :, :, 0, :], kv[:, :, :, 1, :]
    q2 = torch.randn(batch, hq * d, device="cuda", dtype=bf, generator=g)
    k2 = torch.randn(batch, hkv * d, device="cuda", dtype=bf, generator=g)
    v2 = torch.randn(batch, hkv * d, device="cuda", dtype=bf, generator=g)
    qw = torch.ones(d, device="cuda", dtype=bf)
    kw = torch.ones(d, device="cuda", dtype=bf)
    inv = 1e6 ** (-torch.arange(0, d, 2, dtype=torch.float64, device="cuda") / d)
    ang = torch.cat([ctx * inv, ctx * inv]).float().view(1, 1, d)
    cos, sin = ang.cos().to(bf), ang.sin().to(bf)  # the model passes cos/sin in the activation dtype
    pos = torch.tensor([ctx], dtype=torch.long, device="cuda")
    out = torch.empty(batch, hq, d, device="cuda", dtype=bf)
    code = _native.dtype_code
    if not _native.call("qh_flash_decode_prepare_ok", batch, hq, hkv, ctx + 1, d):
        raise RuntimeError("the config-3 decode shape is not served by qh_flash_decode_prepare")

    def launch():
        _native.call("qh_flash_decode_prepare", q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0),
                     v2.data_ptr(), v2.stride(0), qw.data_ptr(), kw.data_ptr(), 1e-6, 0, cos.data_ptr(),
                     sin.data_ptr(), cos.stride(0), 1, d, kc.data_ptr(), *kc.stride()[:3], vc.data_ptr(),
                     *vc.stride()[:3], cap, pos.data_ptr(), out.data_ptr(), None, None, batch, hq, hkv, sk, d,
                     d ** -0.5, code(bf), code(bf), code(bf), _native.stream(torch.device("cuda")))

    kv_bytes = 2 * batch * hkv * sk * d * 2
    rows_bytes = (batch * hq * d + 2 * batch * hkv * d) * 2  # projected q, k, v rows read
    write_bytes = (batch * hq * d + 2 * batch * hkv * d) * 2  # o, new cache rows written
    return launch, kv_bytes + rows_bytes + write_bytes


def attention_roofline(per_graph=20, replays=5):
    """Dominant kernel of the decode step: decode attention with its row preparation over 2049 keys.
    Its launches are captured back to back in a HIP graph (as the step replays them) and timed with
    HIP events around the replays on the stream they run on: average launch = elapsed / launches."""
    import torch

    launch, algo = decode_layer_launch()
    for _ in range(5):
        launch()
    sync()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for _ in range(per_graph):
                launch()
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()
    sync()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(replays):
        graph.replay()
    b.record(stream)
    sync()
    avg_ms = a.elapsed_time(b) / (per_graph * replays)
    achieved = algo / (avg_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": DECODE_TRAFFIC_BYTES,
            "kernel": "fa_decode_wg_kernel<bf16,128,2,PREP>", "avg_launch_us": round(avg_ms * 1e3, 2),
            "algorithmic_bytes_per_launch": algo}


# ---------------------------------------------------------------------------
# config 0 on the GPU: prefill 128, 32 greedy decode steps, batch 1
# ---------------------------------------------------------------------------
# algorithmic work of config 0 (Qwen3-0.6B, bs1): every weight matrix read once per forward
# (28 layers x 31.46 MB + the 311.2 MB tied LM head), the KV cache written once (prefill) or read
# once (decode); prefill flops from the linear layers, attention and the LM head on the last token
CFG0_WEIGHT_BYTES = 28 * 2 * 1024 * (2048 + 1024 + 1024 + 2048 + 3 * 3072) + 2 * 151936 * 1024
CFG0_KV_BYTES_PER_POS = 28 * 2 * 8 * 128 * 2
CFG0_PREFILL_FLOP = 114.95e9


def bench_cfg0(model, reps=5):
    """Config 0 on the GPU: bs1 prefill of 128 tokens and greedy decoding.

    * prefill: a replay of the captured prefill graph (``greedy_graphs``), host-timed around the
      replay with synchronisations; the eager forward beside it;
    * decode: per-token time = (generation of 33 tokens - of 3 tokens) / 30 with
      ``greedy_generate(use_graph=True)``, which cancels the prefill (both graphs are captured
      beforehand, so no capture is timed);
    * roofline of each: algorithmic bytes (weights read once, KV written or read once) over the
      measured time against 8 TB/s, and the prefill's flops against the bf16 MFMA peak."""
    import torch

    ids = torch.randint(0, model.config.vocab_size, (1, 128), generator=torch.Generator().manual_seed(0)).cuda()

    def timed(fn):
        sync()
        t0 = time.perf_counter()
        fn()
        sync()
        return time.perf_counter() - t0

    with torch.no_grad():
        model.greedy_generate(ids, max_new_tokens=3)  # warmup
        for n in (3, 33):
            model.greedy_generate(ids, max_new_tokens=n, use_graph=True)  # captures both shapes
        runner = model.greedy_graphs(1, 128, 33)
        pre_graph = sorted(timed(lambda: runner.prefill(ids)) for _ in range(reps))[reps // 2]
        pre_eager = []
        for _ in range(reps):
            cache = model.new_cache(1, 160, torch.bfloat16, "cuda")
            pre_eager.append(timed(lambda: model(input_ids=ids, past_key_values=cache, use_cache=True,
                                                 logits_to_keep=1).logits[:, -1].argmax(-1)))
        pre_eager = sorted(pre_eager)[reps // 2]
        per_tok = {}
        for name, graph in (("eager", False), ("graph", True)):
            long = min(timed(lambda: model.greedy_generate(ids, max_new_tokens=33, use_graph=graph)) for _ in range(3))
            short = min(timed(lambda: model.greedy_generate(ids, max_new_tokens=3, use_graph=graph)) for _ in range(3))
            per_tok[name] = max(long - short, 1e-9) / 30
    tok = per_tok["graph"]
    pre_bytes = CFG0_WEIGHT_BYTES + 128 * CFG0_KV_BYTES_PER_POS
    dec_bytes = CFG0_WEIGHT_BYTES + 145 * CFG0_KV_BYTES_PER_POS  # mean context of the 30 timed steps
    pre_gbs = pre_bytes / pre_graph / 1e9
    dec_gbs = dec_bytes / tok / 1e9
    return {"prefill_tok_s": round(128 / pre_graph, 1), "prefill_ms": round(pre_graph * 1e3, 3),
            "prefill_mode": "captured prefill graph replayed (greedy_graphs)",
            "prefill_eager_ms": round(pre_eager * 1e3, 3),
            "decode_tok_s": round(1 / tok, 1), "decode_ms_per_token": round(tok * 1e3, 3),
            "decode_mode": "greedy_generate(use_graph=True): captured decode step replayed per token",
            "eager_decode_tok_s": round(1 / per_tok["eager"], 1),
            "roofline": {
                "prefill": {"bound": "hbm", "achieved": round(pre_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(pre_gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": pre_bytes,
                            "mfma_frac": round(CFG0_PREFILL_FLOP / pre_graph / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)},
                "decode_token": {"bound": "hbm", "achieved": round(dec_gbs, 1), "peak": HBM_PEAK_GBS,
                                 "unit": "GB/s", "frac": round(dec_gbs / HBM_PEAK_GBS, 4),
                                 "algorithmic_bytes": dec_bytes}}}


def cpu_baseline_cfg0(model, new_tokens=32):
    """Config 0 on the host cores: the oracle (fp32, HF semantics) prefilling the same 128 ids and
    greedily decoding ``new_tokens`` steps with its KV cache."""
    import torch

    from oracle.model import ModelSpec, OracleQwen

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    params = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    orc = OracleQwen(ModelSpec.from_config(model.config), params, dtype=torch.float32)
    ids = torch.randint(0, model.config.vocab_size, (1, 128), generator=torch.Generator().manual_seed(0))
    orc.forward(ids[:, :16], orc.new_cache(), logits_to_keep=1)  # warmup
    cache = orc.new_cache()
    t0 = time.perf_counter()
    nxt = orc.forward(ids, cache, logits_to_keep=1)[:, -1].argmax(-1, keepdim=True)
    t1 = time.perf_counter()
    for _ in range(new_tokens):
        nxt = orc.forward(nxt, cache, logits_to_keep=1)[:, -1].argmax(-1, keepdim=True)
    t2 = time.perf_counter()
    del params, orc
    return {"prefill_tok_s": round(128 / (t1 - t0), 1), "decode_tok_s": round(new_tokens / (t2 - t1), 2),
            "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"oracle fp32 prefill of the 128 ids ({(t1 - t0) * 1e3:.0f} ms) then {new_tokens} greedy steps "
                      f"({(t2 - t1) * 1e3:.0f} ms), the whole workload"}


# ---------------------------------------------------------------------------
# CPU baseline: the oracle (fp32 torch) on a bounded sample of config 3
# ---------------------------------------------------------------------------
def cpu_baseline(model, sample_batch=4, ctx=2048, reps=3):
    import torch

    from oracle.model import ModelSpec, OracleQwen

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    params = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    orc = OracleQwen(ModelSpec.from_config(model.config), params, dtype=torch.float32)
    cfg = model.config
    gen = torch.Generator().manual_seed(0)
    shape = (sample_batch, cfg.num_key_value_heads, ctx, cfg.head_dim)
    kv = [(torch.randn(shape, generator=gen), torch.randn(shape, generator=gen)) for _ in range(cfg.num_hidden_layers)]
    ids = torch.randint(0, cfg.vocab_size, (sample_batch, 1), generator=gen)

    def run():
        cache = {"k": [a for a, _ in kv], "v": [b for _, b in kv], "len": ctx}
        return orc.forward(ids, cache, logits_to_keep=1)

    run()  # warmup
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
    return {"value": round(sample_batch / t, 2), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"oracle fp32 decode step, batch {sample_batch} of 64, 2048-token cache, 28 layers "
                      f"(median of {reps}, {t:.2f} s/step)"}


# ---------------------------------------------------------------------------
# other configs (profiling workloads)
# ---------------------------------------------------------------------------
def bench_fa(steps, warmup):
    import torch
    from qwen_triton.kernels import flash_attention as FA

    B, Hq, Hkv, S, D = 8, 16, 8, 4096, 128
    g = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(B, Hq, S, D, device="cuda", dtype=torch.bfloat16, generator=g)
    k = torch.randn(B, Hkv, S, D, device="cuda", dtype=torch.bfloat16, generator=g)
    v = torch.randn(B, Hkv, S, D, device="cuda", dtype=torch.bfloat16, generator=g)
    do = torch.randn(B, Hq, S, D, device="cuda", dtype=torch.bfloat16, generator=g)
    scale = D ** -0.5
    for _ in range(warmup):
        o, lse = FA.flash_forward(q, k, v, scale, True, 2)
        FA.flash_backward(q, k, v, o, do, lse, scale, True, 2)
    sync()
    ef, eb = [], []
    for _ in range(steps):
        a, b, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        a.record()
        o, lse = FA.flash_forward(q, k, v, scale, True, 2)
        b.record()
        FA.flash_backward(q, k, v, o, do, lse, scale, True, 2)
        c.record()
        ef.append((a, b))
        eb.append((b, c))
    sync()
    fwd_ms = sum(x.elapsed_time(y) for x, y in ef) / steps
    bwd_ms = sum(x.elapsed_time(y) for x, y in eb) / steps
    fwd_flop = 2 * B * Hq * D * S * (S + 1)
    bwd_flop = 2.5 * fwd_flop

    # Inference forward with the model's masks (qh_flash_fwd_masked): left padding of
    # 0, 1/8, ..., 7/8 of the sequence, and a sliding window of 1024 keys. Flops count the visible
    # (query, key) pairs only: (S - p)(S - p + 1) / 2 per sequence with p padding tokens, and
    # W (W + 1) / 2 + (S - W) W under a window of W.
    pads = [S * i // 8 for i in range(B)]
    valid = torch.ones(B, S, dtype=torch.int64, device="cuda")
    for b, p in enumerate(pads):
        valid[b, :p] = 0
    bits = FA.pack_key_bits(valid)
    W = 1024

    def timed(fn):
        for _ in range(warmup):
            fn()
        sync()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        sync()
        return a.elapsed_time(b) / steps

    pad_ms = timed(lambda: FA.flash_forward(q, k, v, scale, True, 2, need_lse=False, key_bits=bits))
    win_ms = timed(lambda: FA.flash_forward(q, k, v, scale, True, 2, need_lse=False, window=W))
    # A padded decode step at config 3's attention shape (64 sequences, 16 q-heads on 8 kv-heads,
    # 2049 keys, left padding of (13 b) mod 300 tokens) against the unmasked split-KV decode kernel.
    Bd, Hqd, Hkd, Skd = 64, 16, 8, 2049
    qd = torch.randn(Bd, Hqd, 1, D, device="cuda", dtype=torch.bfloat16, generator=g)
    kd = torch.randn(Bd, Hkd, Skd, D, device="cuda", dtype=torch.bfloat16, generator=g)
    vd = torch.randn(Bd, Hkd, Skd, D, device="cuda", dtype=torch.bfloat16, generator=g)
    vdec = torch.ones(Bd, Skd, dtype=torch.int64, device="cuda")
    for b_ in range(Bd):
        vdec[b_, :(13 * b_) % 300] = 0
    bits_d = FA.pack_key_bits(vdec)
    dec_ms = timed(lambda: FA.flash_decode(qd, kd, vd, scale, Hqd // Hkd))
    dec_pad_ms = timed(lambda: FA.flash_forward(qd, kd, vd, scale, True, Hqd // Hkd, Skd - 1, need_lse=False,
                                                key_bits=bits_d))
    pad_flop = 4 * Hq * D * sum((S - p) * (S - p + 1) // 2 for p in pads)
    win_flop = 4 * B * Hq * D * (W * (W + 1) // 2 + (S - W) * W)
    return {"fa_fwd_ms": round(fwd_ms, 3), "fa_bwd_ms": round(bwd_ms, 3),
            "fa_fwd_tflops": round(fwd_flop / fwd_ms / 1e9, 1), "fa_bwd_tflops": round(bwd_flop / bwd_ms / 1e9, 1),
            "fa_fwd_frac": round(fwd_flop / fwd_ms / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4),
            "fa_bwd_frac": round(bwd_flop / bwd_ms / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4),
            "fa_fwd_left_padded_ms": round(pad_ms, 3), "fa_fwd_left_padded_tflops": round(pad_flop / pad_ms / 1e9, 1),
            "fa_fwd_window1024_ms": round(win_ms, 3), "fa_fwd_window1024_tflops": round(win_flop / win_ms / 1e9, 1),
            "decode_attention_us": round(dec_ms * 1e3, 1), "decode_attention_padded_us": round(dec_pad_ms * 1e3, 1)}


def bench_gdr(steps, warmup):
    """Qwen3-Next linear attention's gated delta rule over whole sequences (32 value heads, key and
    value head dims 128, bf16, 4 sequences x 4096 tokens): HIP-event time of one
    `qh_gated_delta_rule` launch, tokens per second, the time per sequential token step, the
    algorithmic bytes (q, k, v read, output written once, decay/beta, final state) over the time,
    and the oracle (fp32 torch on the host cores) on a bounded sample, scaled per (token, head)."""
    import torch
    import torch.nn.functional as F
    from oracle import ops as O
    from qwen_triton.kernels.linear_attention import gated_delta_rule_sequence

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    B, S, H, Dk, Dv = 4, 4096, 32, 128, 128
    g = torch.Generator(device="cuda").manual_seed(0)
    q = F.normalize(torch.randn(B, S, H, Dk, device="cuda", generator=g), dim=-1).bfloat16()
    k = F.normalize(torch.randn(B, S, H, Dk, device="cuda", generator=g), dim=-1).bfloat16()
    v = torch.randn(B, S, H, Dv, device="cuda", generator=g).bfloat16()
    decay = -F.softplus(torch.randn(B, S, H, device="cuda", generator=g)) * 0.5
    beta = torch.sigmoid(torch.randn(B, S, H, device="cuda", generator=g))
    for _ in range(max(1, warmup)):
        gated_delta_rule_sequence(q, k, v, decay, beta)
    sync()
    evs = []
    for _ in range(steps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        gated_delta_rule_sequence(q, k, v, decay, beta)
        b.record()
        evs.append((a, b))
    sync()
    ms = min(x.elapsed_time(y) for x, y in evs)
    nbytes = 2 * (q.numel() + k.numel() + 2 * v.numel()) + 4 * 2 * decay.numel() + 4 * B * H * Dk * Dv
    # oracle: 1 sequence x 128 tokens x 4 heads, fp32, median of 3
    Sc, Hc = 128, 4
    qc, kc, vc = (t[:1, :Sc, :Hc].float().cpu() for t in (q, k, v))
    gc, bc = decay[:1, :Sc, :Hc].cpu(), beta[:1, :Sc, :Hc].cpu()
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        O.gated_delta_rule(qc, kc, vc, gc, bc, dtype=torch.float32)
        ts.append(time.perf_counter() - t0)
    cpu_s = sorted(ts)[1]
    cpu_tok_s = Sc * Hc / cpu_s / H  # tokens of all 32 heads per second
    return {"gdr_ms": round(ms, 3), "tokens": B * S, "heads": H, "gdr_tok_s": round(B * S / ms * 1e3, 1),
            "us_per_token_step": round(ms * 1e3 / S, 3), "gbs": round(nbytes / ms / 1e6, 1),
            "hbm_frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
            "cpu_baseline": {"value": round(cpu_tok_s, 1), "unit": "tok/s (all 32 heads)",
                             "cores": torch.get_num_threads(), "kind": "port",
                             "sample": f"oracle fp32 gated delta rule, 1 sequence x {Sc} tokens x {Hc} heads "
                                       f"({cpu_s * 1e3:.1f} ms), scaled per (token, head)"}}


def bench_dense(steps, warmup):
    import torch
    from qwen_triton.kernels import cross_entropy as CE
    from qwen_triton.kernels import matmul as MM
    from qwen_triton.kernels import silu_mul

    T, H, I, V = 16384, 1024, 3072, 151936
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(T, H, device="cuda", dtype=torch.bfloat16, generator=g).requires_grad_(True)
    wg = (torch.randn(I, H, device="cuda", generator=g) * 0.02).bfloat16().requires_grad_(True)
    wu = (torch.randn(I, H, device="cuda", generator=g) * 0.02).bfloat16().requires_grad_(True)
    wd = (torch.randn(H, I, device="cuda", generator=g) * 0.02).bfloat16().requires_grad_(True)
    wl = (torch.randn(V, H, device="cuda", generator=g) * 0.02).bfloat16().requires_grad_(True)
    labels = torch.randint(0, V, (T,), device="cuda", generator=g)

    from qwen_triton.kernels import fused_linear_cross_entropy

    def step(fused=False):
        for t in (x, wg, wu, wd, wl):  # released as optimizer.zero_grad(set_to_none=True) does each step
            t.grad = None
        h = MM.triton_matmul(silu_mul(MM.triton_matmul(x, wg), MM.triton_matmul(x, wu)), wd)
        if fused:  # LM head + CE without the [16384, 151936] logits (recomputed per vocabulary chunk)
            loss = fused_linear_cross_entropy(h, wl, labels)
        else:
            loss = CE.triton_cross_entropy(MM.triton_matmul(h, wl), labels)
        loss.backward()
        return loss

    res = {}
    flop = 3 * (3 * 2 * T * H * I + 2 * T * H * V)
    for fused in (False, True):
        for _ in range(warmup):
            step(fused)
        sync()
        torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        for _ in range(steps):
            step(fused)
        sync()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        key = "dense_fused_ce" if fused else "dense"
        res[f"{key}_ms_per_step"] = round(ms, 3)
        res[f"{key}_gemm_tflops"] = round(flop / ms / 1e9, 1)
        res[f"{key}_gemm_frac_of_step"] = round(flop / ms / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4)
        res[f"{key}_peak_mem_gb"] = round(torch.cuda.max_memory_allocated() / 1e9, 2)
    # the fused backward recomputes the LM-head logits (one more 16384 x 151936 x 1024 product), so its
    # GEMM flop count is higher than `flop`; the rates above use the unfused count for both
    return res


def bench_gemm(steps, warmup, only=None):
    """Per-shape GEMM timing (HIP events): ours vs torch.matmul (hipBLASLt) for context."""
    import torch
    from qwen_triton.kernels import matmul as MM

    shapes = [  # (label, layout, M, N, K)
        ("decode q", "NT", 64, 2048, 1024), ("decode kv", "NT", 64, 1024, 1024), ("decode gate", "NT", 64, 3072, 1024),
        ("decode down", "NT", 64, 1024, 3072), ("decode lm_head", "NT", 64, 151936, 1024),
        ("bs1 lm_head", "NT", 1, 151936, 1024), ("bs1 gate", "NT", 1, 3072, 1024),
        ("prefill128 q", "NT", 128, 2048, 1024), ("prefill128 gate", "NT", 128, 3072, 1024),
        ("prefill128 down", "NT", 128, 1024, 3072),
        ("train gate fwd", "NT", 16384, 3072, 1024), ("train down fwd", "NT", 16384, 1024, 3072),
        ("train lm_head fwd", "NT", 16384, 151936, 1024), ("train down dX", "NN", 16384, 3072, 1024),
        ("train gate dW", "TN", 3072, 1024, 16384), ("square 8192", "NT", 8192, 8192, 8192),
    ]
    if only:
        shapes = [sh for sh in shapes if sh[0] == only]
    g = torch.Generator(device="cuda").manual_seed(0)
    out = []
    for label, lay, M, N, K in shapes:
        if lay == "NT":
            a = torch.randn(M, K, device="cuda", dtype=torch.bfloat16, generator=g)
            b = torch.randn(N, K, device="cuda", dtype=torch.bfloat16, generator=g)
            ours = lambda: MM.gemm(False, False, M, N, K, a, K, b, K, c, N)
            ref = lambda: torch.matmul(a, b.T)
        elif lay == "NN":
            a = torch.randn(M, K, device="cuda", dtype=torch.bfloat16, generator=g)
            b = torch.randn(K, N, device="cuda", dtype=torch.bfloat16, generator=g)
            ours = lambda: MM.gemm(False, True, M, N, K, a, K, b, N, c, N)
            ref = lambda: torch.matmul(a, b)
        else:
            a = torch.randn(K, M, device="cuda", dtype=torch.bfloat16, generator=g)
            b = torch.randn(K, N, device="cuda", dtype=torch.bfloat16, generator=g)
            ours = lambda: MM.gemm(True, True, M, N, K, a, M, b, N, c, N)
            ref = lambda: torch.matmul(a.T, b)
        c = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        # Both are warmed up, then timed in alternating rounds (clocks ramp and settle over the
        # first tens of milliseconds of a large product); each keeps its best round's mean.
        res = {"ours": float("inf"), "torch": float("inf")}
        for fn in (ours, ref):
            for _ in range(warmup):
                fn()
        for _ in range(3):
            for name, fn in (("ours", ours), ("torch", ref)):
                evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                       for _ in range(steps)]
                for e0, e1 in evs:
                    e0.record()
                    fn()
                    e1.record()
                sync()
                res[name] = min(res[name], sum(e0.elapsed_time(e1) for e0, e1 in evs) / steps)
        flop = 2 * M * N * K
        nbytes = 2 * (M * K + N * K + M * N)
        row = {"shape": label, "layout": lay, "M": M, "N": N, "K": K, "us": round(res["ours"] * 1e3, 2),
               "tflops": round(flop / res["ours"] / 1e9, 1), "gbs": round(nbytes / res["ours"] / 1e6, 1),
               "torch_us": round(res["torch"] * 1e3, 2)}
        log(json.dumps(row))
        out.append(row)
    return out


def bench_moe(steps, warmup, loop_reps=1):
    """Config 4: one Qwen3-MoE layer at 30B-A3B shape on 16384 bf16 tokens (4 x 4096, causal).

    Times (HIP events, inputs resident): the expert path forward without autograd (routing +
    dispatch + grouped GEMMs + combine), the expert path forward + backward with autograd
    (router logits, input and every expert weight get gradients), and the whole decoder layer
    (RMSNorm, attention, MoE block) forward + backward. Each training step first releases the
    previous step's gradients (zero_grad(set_to_none=True), as a training loop does), so it writes
    fresh gradients instead of adding into old ones. The reference's per-expert loop is timed once
    beside them."""
    import torch
    from qwen_triton import QwenTritonConfig
    from qwen_triton.models.core import QwenDecoderLayer
    from qwen_triton.modules.rotary import QwenRotaryEmbedding

    B, S, H, E, K, I = 4, 4096, 2048, 128, 8, 768
    T = B * S
    cfg = QwenTritonConfig.from_hf_config(dict(
        model_type="qwen3_moe", vocab_size=151936, hidden_size=H, intermediate_size=6144, num_hidden_layers=1,
        num_attention_heads=32, num_key_value_heads=4, head_dim=128, moe_intermediate_size=I, num_experts=E,
        num_experts_per_tok=K, norm_topk_prob=True, decoder_sparse_step=1, mlp_only_layers=[]))
    torch.manual_seed(0)
    layer = QwenDecoderLayer(cfg, 0)
    with torch.no_grad():
        for n, prm in layer.named_parameters():
            if "norm" in n:
                prm.fill_(1.0)
            else:
                prm.normal_(0.0, 0.02)
    layer = layer.to("cuda", torch.bfloat16)
    blk = layer.mlp
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(T, H, device="cuda", dtype=torch.bfloat16, generator=g)
    logits = torch.randn(T, E, device="cuda", dtype=torch.float32, generator=g)
    go = torch.randn(T, H, device="cuda", dtype=torch.bfloat16, generator=g)

    def timed(fn, n, w):
        for _ in range(w):
            fn()
        sync()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        sync()
        return e0.elapsed_time(e1) / n

    def infer():
        w, sel = blk.route(logits, torch.bfloat16)
        return blk.experts_forward(x, w, sel)

    xg = x.clone().requires_grad_(True)
    lg = logits.clone().requires_grad_(True)

    def train():
        blk.zero_grad(set_to_none=True)  # a training loop's per-step release: no accumulation into old grads
        xg.grad = lg.grad = None
        w, sel = blk.route(lg, torch.bfloat16)
        out = blk.experts_forward(xg, w, sel)
        torch.autograd.backward(out, go)

    with torch.no_grad():
        ms_inf = timed(infer, steps, warmup)
    ms_train = timed(train, steps, warmup)
    flop = 2 * 3 * T * K * H * I  # gate, up, down over the T*K routed rows
    res = {"moe_fwd_ms": round(ms_inf, 3), "moe_fwd_tflops": round(flop / ms_inf / 1e9, 1),
           "moe_fwd_frac": round(flop / ms_inf / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4),
           "moe_fwd_bwd_ms": round(ms_train, 3), "moe_fwd_bwd_tflops": round(3 * flop / ms_train / 1e9, 1),
           "moe_fwd_bwd_frac": round(3 * flop / ms_train / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4),
           "tokens": T, "experts": E, "top_k": K}

    rot = QwenRotaryEmbedding(cfg).to("cuda")
    pos = torch.arange(S, device="cuda")[None].expand(B, S)
    hs = torch.randn(B, S, H, device="cuda", dtype=torch.bfloat16, generator=g).requires_grad_(True)
    gl = torch.randn(B, S, H, device="cuda", dtype=torch.bfloat16, generator=g)
    cos, sin = rot(hs, pos)

    def layer_step():
        layer.zero_grad(set_to_none=True)
        hs.grad = None
        out, _ = layer(hs, (cos, sin))
        torch.autograd.backward(out, gl)

    ms_layer = timed(layer_step, steps, warmup)
    res["layer_fwd_bwd_ms"] = round(ms_layer, 3)
    res["layer_tokens_per_s"] = round(T / ms_layer * 1e3, 1)

    if loop_reps <= 0:
        return res
    # the reference's per-expert loop (forward + backward), once
    saved = blk._grouped_ok
    blk._grouped_ok = lambda *a, **kw: False
    try:
        sync()
        t0 = time.perf_counter()
        for _ in range(loop_reps):
            train()
        sync()
        res["loop_fwd_bwd_ms"] = round((time.perf_counter() - t0) * 1e3 / loop_reps, 3)
    finally:
        blk._grouped_ok = saved
    return res


def bench_ops(reps=20):
    """Per-operator measurement at config shapes: HIP-event time, achieved GB/s against the HBM
    roofline, and the oracle (fp32 torch on the host cores) on a bounded row sample beside it."""
    import torch
    from oracle import ops as O
    from qwen_triton import kernels as K

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    cores = torch.get_num_threads()
    g = torch.Generator(device="cuda").manual_seed(0)
    bf = torch.bfloat16

    def rnd(*shape, dtype=bf, scale=1.0):
        return (torch.randn(*shape, device="cuda", generator=g) * scale).to(dtype)

    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    torch.cuda._sleep(10_000_000)
    ev1.record()
    sync()
    cycles_per_ms = 10_000_000 / ev0.elapsed_time(ev1)

    def gpu_ms(fn, n=reps):
        """Device time per call: the timed launches are queued behind a spin kernel sized to
        outlast their host-side enqueue, so they run back to back on the GPU."""
        fn()
        sync()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        sync()
        host_ms = (time.perf_counter() - t0) * 1e3
        torch.cuda._sleep(int(cycles_per_ms * (1.5 * host_ms + 1.0)))
        ev0.record()
        for _ in range(n):
            fn()
        ev1.record()
        sync()
        return ev0.elapsed_time(ev1) / n

    def cpu_ms(fn, n=3):
        fn()
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2] * 1e3

    rows = []

    def record(row, op, shape, ms, nbytes, rows_gpu, cpu_fn=None, rows_cpu=None):
        r = {"row": row, "op": op, "shape": shape, "gpu_us": round(ms * 1e3, 2),
             "gbs": round(nbytes / ms / 1e6, 1), "hbm_frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 3)}
        if cpu_fn is not None:
            c = cpu_ms(cpu_fn)
            r["cpu_sample_rows"] = rows_cpu
            r["cpu_ms"] = round(c, 2)
            r["gpu_vs_cpu_per_row"] = round((c / rows_cpu) / (ms / rows_gpu), 1)
        log(json.dumps(r))
        rows.append(r)

    f32 = torch.float32
    # a2 embedding (16384 tokens of the 151936 x 1024 table), fwd and bwd (full dW written)
    T, H, V = 16384, 1024, 151936
    w = rnd(V, H, scale=0.02)
    ids = torch.randint(0, V, (T,), device="cuda", generator=g)
    ms = gpu_ms(lambda: K.triton_embedding(ids, w))
    record("a2", "embedding fwd", [T, H], ms, 2 * T * H * 2 + T * 8, T,
           lambda: O.embedding(ids[:2048].cpu(), w.float().cpu(), dtype=f32), 2048)
    wg = w.clone().requires_grad_(True)
    go = rnd(T, H)
    ms_fb = gpu_ms(lambda: torch.autograd.grad(K.triton_embedding(ids, wg), wg, go), 5)
    ms_f = gpu_ms(lambda: K.triton_embedding(ids, wg), 5)
    record("a2", "embedding bwd", [T, H], ms_fb - ms_f, T * H * 2 + V * H * 2 + T * 8, T,
           lambda: O.embedding_backward(ids[:2048].cpu(), go[:2048].float().cpu(), V, dtype=f32), 2048)
    # a4 rmsnorm at 16384 x 1024 (config 2) and 16384 x 2048 (config 4), fwd and bwd
    for C in (1024, 2048):
        x = rnd(T, C)
        wn = torch.ones(C, device="cuda", dtype=bf)
        ms = gpu_ms(lambda: K.rmsnorm(x, wn))
        record("a4", "rmsnorm fwd", [T, C], ms, 2 * T * C * 2, T,
               lambda: O.rmsnorm(x[:2048].cpu(), wn.cpu(), dtype=f32), 2048)
        xg = x.clone().requires_grad_(True)
        wq = wn.clone().requires_grad_(True)
        gy = rnd(T, C)
        ms_fb = gpu_ms(lambda: torch.autograd.grad(K.rmsnorm(xg, wq), (xg, wq), gy), 10)
        ms_f = gpu_ms(lambda: K.rmsnorm(xg, wq), 10)
        record("a4", "rmsnorm bwd", [T, C], ms_fb - ms_f, 3 * T * C * 2, T,
               lambda: O.rmsnorm_backward(x[:2048].cpu(), wn.cpu(), gy[:2048].cpu(), dtype=f32), 2048)
    # a5 RoPE on config-1 q and k ([8,16,4096,128] / [8,8,4096,128]), cos/sin [1,4096,128]
    q = rnd(8, 16, 4096, 128)
    k = rnd(8, 8, 4096, 128)
    pos = torch.arange(4096, device="cuda")
    cos, sin = O.rotary_tables(pos, 128, 1e6)
    cos, sin = cos.to("cuda", bf), sin.to("cuda", bf)
    ms = gpu_ms(lambda: K.apply_rope(q, k, cos, sin))
    nq = q.numel() + k.numel()
    record("a5", "apply_rope (q and k)", [8, 24, 4096, 128], ms, 2 * nq * 2, 8 * 24 * 4096,
           lambda: O.rope(q[:1, :, :512].cpu(), cos[:, :512].cpu(), sin[:, :512].cpu(), dtype=f32), 16 * 512)
    # a6 silu_mul and a7 sigmoid_mul at [16384, 3072] / [16384, 2048], fwd and bwd
    for row, name, fn, ofn, ofb, C in (("a6", "silu_mul", K.silu_mul, O.silu_mul, O.silu_mul_backward, 3072),
                                       ("a7", "sigmoid_mul", K.sigmoid_mul, O.sigmoid_mul, O.sigmoid_mul_backward,
                                        2048)):
        a, b2 = rnd(T, C), rnd(T, C)
        ms = gpu_ms(lambda: fn(a, b2))
        record(row, f"{name} fwd", [T, C], ms, 3 * T * C * 2, T, lambda: ofn(a[:2048].cpu(), b2[:2048].cpu(), dtype=f32),
               2048)
        ag, bg = a.clone().requires_grad_(True), b2.clone().requires_grad_(True)
        go2 = rnd(T, C)
        ms_fb = gpu_ms(lambda: torch.autograd.grad(fn(ag, bg), (ag, bg), go2), 10)
        ms_f = gpu_ms(lambda: fn(ag, bg), 10)
        record(row, f"{name} bwd", [T, C], ms_fb - ms_f, 5 * T * C * 2, T,
               lambda: ofb(a[:2048].cpu(), b2[:2048].cpu(), go2[:2048].cpu(), dtype=f32), 2048)
    # a15 residual add [16384, 1024]
    x1, x2 = rnd(T, H), rnd(T, H)
    ms = gpu_ms(lambda: K.residual_add(x1, x2))
    record("a15", "residual_add", [T, H], ms, 3 * T * H * 2, T,
           lambda: O.residual_add(x1[:2048].cpu(), x2[:2048].cpu(), dtype=f32), 2048)
    # a8 KV cache write: config-3 decode step (64 x 8 x 1 x 128 into cap 4096) and a 4096-token prefill
    for S in (1, 4096):
        Bc = 64 if S == 1 else 1
        cache = rnd(Bc, 8, 4096, 128)
        vals = rnd(Bc, 8, S, 128)
        p_ = torch.arange(S, device="cuda") + (2048 if S == 1 else 0)
        ms = gpu_ms(lambda: K.write_attention_kv(cache, vals, p_))
        record("a8", f"write_attention_kv S={S}", [Bc, 8, S, 128], ms, 2 * vals.numel() * 2, Bc * 8 * S,
               lambda: O.kv_write(cache[:1].cpu(), vals[:1].cpu(), p_.cpu()), 8 * S)
    # a9 cross-entropy over [16384, 151936] bf16 logits, fwd and bwd
    logits = rnd(T, V)
    tgt = torch.randint(0, V, (T,), device="cuda", generator=g)
    ms = gpu_ms(lambda: K.triton_cross_entropy(logits, tgt), 5)
    record("a9", "cross_entropy fwd", [T, V], ms, T * V * 2, T,
           lambda: O.cross_entropy(logits[:64].cpu(), tgt[:64].cpu(), dtype=f32), 64)
    lg = logits.clone().requires_grad_(True)
    ms_fb = gpu_ms(lambda: torch.autograd.grad(K.triton_cross_entropy(lg, tgt), lg), 3)
    ms_f = gpu_ms(lambda: K.triton_cross_entropy(lg, tgt), 3)
    record("a9", "cross_entropy bwd", [T, V], ms_fb - ms_f, 2 * T * V * 2, T,
           lambda: O.cross_entropy_backward(logits[:64].cpu(), tgt[:64].cpu(), dtype=f32), 64)
    del logits, lg
    # MoE routing at config 4: router logits [16384, 128] fp32, top-8
    E, KK = 128, 8
    rl = torch.randn(T, E, device="cuda", generator=g)
    ms = gpu_ms(lambda: K.triton_softmax(rl))
    record("a10", "softmax fwd", [T, E], ms, 2 * T * E * 4, T, lambda: O.softmax(rl[:2048].cpu(), dtype=f32), 2048)
    rg = rl.clone().requires_grad_(True)
    gs = torch.randn(T, E, device="cuda", generator=g)
    ms_fb = gpu_ms(lambda: torch.autograd.grad(K.triton_softmax(rg), rg, gs), 10)
    ms_f = gpu_ms(lambda: K.triton_softmax(rg), 10)
    ys = K.triton_softmax(rl)
    record("a10", "softmax bwd", [T, E], ms_fb - ms_f, 3 * T * E * 4, T,
           lambda: O.softmax_backward(ys[:2048].cpu(), gs[:2048].cpu(), dtype=f32), 2048)
    probs = K.triton_softmax(rl)
    ms = gpu_ms(lambda: K.triton_topk(probs, KK))
    record("a11", "topk k=8", [T, E], ms, T * E * 4 + T * KK * 12, T, lambda: O.topk(probs[:2048].cpu(), KK), 2048)
    sel = K.triton_topk(probs, KK)[1]
    ms = gpu_ms(lambda: K.triton_one_hot(sel, E))
    record("a12", "one_hot", [T, KK, E], ms, T * KK * 8 + T * KK * E * 8, T,
           lambda: O.one_hot(sel[:2048].cpu(), E), 2048)
    # a13 index_add: one expert's share (1024 routed rows of 2048) into the [16384, 2048] target
    tgt2 = rnd(T, 2048)
    src = rnd(1024, 2048)
    idx = torch.randint(0, T, (1024,), device="cuda", generator=g)
    ms = gpu_ms(lambda: K.triton_index_add(tgt2, src, idx))
    record("a13", "index_add (1024 rows into 16384)", [T, 2048], ms, 3 * 1024 * 2048 * 2, 1024,
           lambda: O.index_add(tgt2[:4096].cpu(), src[:256].cpu(), (idx[:256] % 4096).cpu(), dtype=f32), 256)
    # floors of the small launches above, timed the same way: an empty kernel back to back, and
    # torch's device copy of the same bytes as softmax fwd and the S=4096 KV write (8.4 MB each way)
    ms = gpu_ms(lambda: torch.cuda._sleep(0))
    record("floor", "empty launch", [], ms, 0, 1)
    cs, cd = torch.empty(T * E, device="cuda"), torch.empty(T * E, device="cuda")
    ms = gpu_ms(lambda: cd.copy_(cs))
    record("floor", "device copy 8.4 MB", [T * E], ms, 2 * T * E * 4, 1)
    return {"cpu_cores": cores, "rows": rows}


def bench_roofline_kernels(reps=20):
    """Only the dominant decode kernel (one layer of the step) plus a 1 GiB copy for counter calibration."""
    import torch

    launch, algo = decode_layer_launch()
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    times = {"decode": [], "copy": []}
    for i in range(reps):
        for name, fn in (("decode", launch), ("copy", lambda: dst.copy_(src))):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            times[name].append((a, b))
    sync()
    res = {k: sum(a.elapsed_time(b) for a, b in v[2:]) / (len(v) - 2) * 1e3 for k, v in times.items()}
    return {"decode_us": round(res["decode"], 2), "decode_gbs": round(algo / res["decode"] / 1e3, 1),
            "copy_us": round(res["copy"], 2), "copy_gbs": round(2 * (1 << 30) / res["copy"] / 1e3, 1),
            "decode_algorithmic_bytes": algo, "copy_bytes_each_way": 1 << 30}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "fa", "dense", "gemm", "roofline", "moe", "ops", "gdr"])
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--gemm-shape", default=None, help="--workload gemm: time only the shape with this label")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true", help="default run: skip the config 1/2/4 keys")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the kernels run on one "
              "GPU's share of the work); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    os.environ.setdefault("QWEN_TRITON_STRICT", "1")
    import torch
    from qwen_triton import _native

    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    if not _native.available():
        sys.exit(f"libqwen_hip.so not loadable: {_native.load_error()!r}")

    if args.workload == "fa":
        res = bench_fa(args.steps, args.warmup)
        print(json.dumps({"metric": "flash attention fwd+bwd (config 1)", **res}), flush=True)
        return
    if args.workload == "roofline":
        print(json.dumps({"metric": "dominant kernel + calibration copy", **bench_roofline_kernels()}), flush=True)
        return
    if args.workload == "gemm":
        res = bench_gemm(args.steps, args.warmup, args.gemm_shape)
        print(json.dumps({"metric": "GEMM shapes (bf16)", "rows": res}), flush=True)
        return
    if args.workload == "ops":
        res = bench_ops()
        print(json.dumps({"metric": "per-operator HBM throughput at config shapes (+ oracle on host cores)",
                          **res}), flush=True)
        return
    if args.workload == "moe":
        res = bench_moe(args.steps, args.warmup)
        print(json.dumps({"metric": "Qwen3-MoE layer fwd/bwd (config 4, 30B-A3B shape)", **res}), flush=True)
        return
    if args.workload == "gdr":
        res = bench_gdr(args.steps, args.warmup)
        print(json.dumps({"metric": "Qwen3-Next gated delta rule (4 x 4096 tokens, 32 heads, 128/128)", **res}),
              flush=True)
        return
    if args.workload == "dense":
        res = bench_dense(args.steps, args.warmup)
        print(json.dumps({"metric": "dense proj + LM head + CE fwd/bwd (config 2)", **res}), flush=True)
        return

    # the dominant kernel first, on fresh allocations (after the 15 GB decode cache has been
    # allocated and freed the same launches time 3-4 us slower)
    roof = attention_roofline()
    log(f"decode attention: {roof['avg_launch_us']} us/launch, {roof['achieved']} GB/s")
    torch.cuda.empty_cache()
    log("building Qwen3-0.6B (random N(0,0.02) weights, bf16)")
    model = build_model(torch.bfloat16, "cuda")
    cache, eager_ms, graph_ms = bench_decode(model, args.steps, args.warmup, use_graph=not args.no_graph)
    del cache
    torch.cuda.empty_cache()
    cfg0 = bench_cfg0(model)
    log(f"config 0: {cfg0}")
    cpu = None if args.no_cpu_baseline else cpu_baseline(model)
    if cpu:
        log(f"cpu baseline: {cpu}")
        cfg0["cpu_baseline"] = cpu_baseline_cfg0(model)
        log(f"config 0 cpu baseline: {cfg0['cpu_baseline']}")
    del model
    torch.cuda.empty_cache()
    others = {}
    if not args.no_other_configs:
        # the other BASELINE configs' kernels, timed compactly (HIP events / host clock around synchronised steps).
        # Each phase starts on a GPU that idled while the host built it: three warm-up steps and ten timed
        # ones (the first steps after an idle gap run slower; config 4's expert path measured 6.4-6.5 ms
        # over 3 steps after 1 warm-up against 5.36 over 10 after 3)
        others["config1_fa"] = bench_fa(10, 3)
        log(f"config 1: {others['config1_fa']}")
        torch.cuda.empty_cache()
        others["config2_dense"] = bench_dense(10, 3)
        log(f"config 2: {others['config2_dense']}")
        torch.cuda.empty_cache()
        others["config4_moe"] = bench_moe(10, 3, loop_reps=0)
        log(f"config 4: {others['config4_moe']}")
        torch.cuda.empty_cache()
    ms = graph_ms if graph_ms is not None else eager_ms
    line = {
        "metric": METRIC,
        "value": round(64 / (ms * 1e-3), 1),
        "unit": "decode tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random N(0,0.02) weights (seed 0), N(0,1) bf16 KV cache, random token ids",
        "config": {"workload": "config3: Qwen3-0.6B decode step, batch 64, 2048-token KV cache, position 2048, "
                               "28 layers, HIP-graph replay",
                   "global_batch": 64, "seq_len": 2049, "parallelism": "single GPU"},
        "eager_ms_per_step": round(eager_ms, 4),
        "prefill_tok_s": cfg0["prefill_tok_s"],
        "config0_gpu": cfg0,
        **others,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
