"""Model-level parity on CPU (the reference's tests/test_model_parity.py and
tests/test_config.py, restated), plus the golden HF fixtures.

On CPU tensors every operator takes its torch path, exactly like the
reference's own CPU parity tests; the GPU model tests live in
test_gpu_model.py.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.model import ModelSpec, OracleQwen
from qwen_triton import QwenTritonConfig, QwenTritonForCausalLM
from qwen_triton.loaders.hf import _expand_fused

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load_golden(name: str):
    d = np.load(GOLDEN / name, allow_pickle=False)
    params = {k[len("param/"):]: torch.from_numpy(d[k]) for k in d.files if k.startswith("param/")}
    cfg = {k: v for k, v in zip(d["config_keys"].tolist(), d["config_values"].tolist())}
    return params, torch.from_numpy(d["ids"]), torch.from_numpy(d["logits"]), cfg


def _our_config(cfg: dict, moe: bool) -> QwenTritonConfig:
    raw = {k: (int(v) if float(v).is_integer() and k not in ("rope_theta", "rms_norm_eps") else v) for k, v in cfg.items()}
    raw["model_type"] = "qwen3_moe" if moe else "qwen3"
    raw["tie_word_embeddings"] = bool(raw["tie_word_embeddings"])
    if moe:
        raw["norm_topk_prob"] = bool(raw["norm_topk_prob"])
        raw["mlp_only_layers"] = []
    return QwenTritonConfig.from_hf_config(raw)


def _converted(params: dict) -> dict:
    out = {}
    for k, v in params.items():
        out.update(_expand_fused(k, v))
    return out


@pytest.mark.parametrize("name,moe", [("qwen3_tiny.npz", False), ("qwen3_moe_tiny.npz", True)])
def test_golden_logits_oracle_and_model(name, moe):
    params, ids, logits, cfg = _load_golden(name)
    config = _our_config(cfg, moe)
    sd = _converted(params)
    orc = OracleQwen(ModelSpec.from_config(config), sd, dtype=torch.float32)
    torch.testing.assert_close(orc.forward(ids), logits, atol=1e-5, rtol=1e-4)
    model = QwenTritonForCausalLM.from_config(config).eval()
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not missing and not unexpected
    with torch.no_grad():
        ours = model(input_ids=ids, attention_mask=torch.ones_like(ids), use_cache=False).logits
    torch.testing.assert_close(ours, logits, atol=1e-5, rtol=1e-4)


def _tiny_dense():
    from transformers.models.qwen3.configuration_qwen3 import Qwen3Config

    return Qwen3Config(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=16, max_position_embeddings=64,
                       tie_word_embeddings=False)


def test_qwen3_dense_tiny_parity_with_hf():
    # reference tests/test_model_parity.py:18-39
    from transformers.models.qwen3.modeling_qwen3 import Qwen3ForCausalLM

    torch.manual_seed(0)
    cfg = _tiny_dense()
    hf = Qwen3ForCausalLM(cfg).eval()
    ours = QwenTritonForCausalLM.from_config(cfg).eval()
    missing, unexpected = ours.load_state_dict(hf.state_dict(), strict=False)
    assert not missing and not unexpected
    ids = torch.randint(0, cfg.vocab_size, (2, 8))
    with torch.no_grad():
        a = hf(input_ids=ids, attention_mask=torch.ones_like(ids), use_cache=False).logits
        b = ours(input_ids=ids, attention_mask=torch.ones_like(ids), use_cache=False).logits
    torch.testing.assert_close(b, a, atol=1e-5, rtol=1e-4)


def test_cached_decode_matches_full_forward():
    # reference tests/test_model_parity.py:42-80
    torch.manual_seed(0)
    ours = QwenTritonForCausalLM.from_config(_tiny_dense()).eval()
    prompt = torch.randint(0, 128, (1, 5))
    nxt = torch.randint(0, 128, (1, 1))
    full = torch.cat((prompt, nxt), dim=-1)
    with torch.no_grad():
        p = ours(input_ids=prompt, attention_mask=torch.ones_like(prompt), use_cache=True)
        assert p.past_key_values.get_seq_length() == 5
        c = ours(input_ids=nxt, attention_mask=torch.ones_like(full), past_key_values=p.past_key_values,
                 use_cache=True, logits_to_keep=1)
        f = ours(input_ids=full, attention_mask=torch.ones_like(full), use_cache=False, logits_to_keep=1)
    torch.testing.assert_close(c.logits, f.logits, atol=1e-5, rtol=1e-4)
    assert c.past_key_values.get_seq_length() == 6
    assert c.past_key_values.key_cache[0].shape[-2] >= 6


def test_padding_mask_path_matches_oracle_on_unpadded_rows():
    torch.manual_seed(0)
    ours = QwenTritonForCausalLM.from_config(_tiny_dense()).eval()
    ids = torch.randint(0, 128, (2, 6))
    mask = torch.ones_like(ids)
    mask[1, :2] = 0  # left padding on row 1
    with torch.no_grad():
        out = ours(input_ids=ids, attention_mask=mask, use_cache=False).logits
        ref = ours(input_ids=ids[:1], use_cache=False).logits
    torch.testing.assert_close(out[:1], ref, atol=1e-5, rtol=1e-4)


def test_greedy_generate_matches_oracle():
    torch.manual_seed(0)
    ours = QwenTritonForCausalLM.from_config(_tiny_dense()).eval()
    ids = torch.randint(0, 128, (1, 7))
    gen = ours.greedy_generate(ids, max_new_tokens=5)
    orc = OracleQwen(ModelSpec.from_config(ours.config), ours.state_dict()).greedy_generate(ids, 5)
    assert torch.equal(gen, orc)


def test_training_loss_matches_oracle_cross_entropy():
    from oracle import ops as O

    torch.manual_seed(0)
    ours = QwenTritonForCausalLM.from_config(_tiny_dense())
    ids = torch.randint(0, 128, (2, 9))
    out = ours(input_ids=ids, labels=ids)
    exp = O.cross_entropy(out.logits[:, :-1].reshape(-1, 128), ids[:, 1:].reshape(-1))[0]
    torch.testing.assert_close(out.loss.double(), exp, atol=1e-6, rtol=1e-6)
    out.loss.backward()
    assert ours.model.embed_tokens.weight.grad is not None


def test_qwen35_text_config_normalization():
    # reference tests/test_config.py:4-35
    raw = {"model_type": "qwen3_5_moe", "text_config": {
        "model_type": "qwen3_5_moe_text", "vocab_size": 32000, "hidden_size": 128, "intermediate_size": 256,
        "num_hidden_layers": 4, "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 32,
        "max_position_embeddings": 4096, "rms_norm_eps": 1e-6, "attn_output_gate": True,
        "partial_rotary_factor": 0.25, "linear_conv_kernel_dim": 4, "linear_key_head_dim": 16,
        "linear_value_head_dim": 16, "linear_num_key_heads": 4, "linear_num_value_heads": 4, "num_experts": 8,
        "num_experts_per_tok": 2, "moe_intermediate_size": 64, "shared_expert_intermediate_size": 64,
        "layer_types": ["linear_attention", "full_attention", "linear_attention", "full_attention"]}}
    c = QwenTritonConfig.from_hf_config(raw)
    assert c.family == "qwen35_text_moe" and c.norm_one_plus is True and c.rotary_dim == 8
    assert c.layer_types[0] == "linear_attention"


def test_qwen3_dense_normalization():
    # reference tests/test_config.py:39-53
    c = QwenTritonConfig.from_hf_config({"model_type": "qwen3", "vocab_size": 32000, "hidden_size": 128,
                                         "intermediate_size": 256, "num_hidden_layers": 2, "num_attention_heads": 4,
                                         "num_key_value_heads": 2, "head_dim": 32})
    assert c.family == "qwen3_dense" and c.norm_one_plus is False
    assert c.layer_types == ["full_attention", "full_attention"]


def test_hf5_config_rope_parameters_are_read():
    c = QwenTritonConfig.from_hf_config(_tiny_dense())
    assert c.rope_theta == 10000.0 and c.head_dim == 16 and c.num_key_value_heads == 2


def _next_model():
    params, ids, logits, cfg = _load_golden("qwen3_next_tiny.npz")
    raw = {k: (int(v) if float(v).is_integer() and k not in ("rope_theta", "rms_norm_eps", "partial_rotary_factor")
               else v) for k, v in cfg.items()}
    raw["model_type"] = "qwen3_next"
    raw["tie_word_embeddings"] = bool(raw["tie_word_embeddings"])
    raw["norm_topk_prob"] = bool(raw["norm_topk_prob"])
    raw["mlp_only_layers"] = []
    config = QwenTritonConfig.from_hf_config(raw)
    assert config.layer_types == ["linear_attention", "full_attention"] * 2
    model = QwenTritonForCausalLM.from_config(config).eval()
    missing, unexpected = model.load_state_dict(_converted(params), strict=False)
    assert not missing and not unexpected, (missing, unexpected)
    return model, ids, logits


def test_golden_qwen3_next_logits_and_cached_decode():
    """Qwen3-Next (gated-delta linear attention + gated full attention, partial rotary, (1+w) norms,
    MoE with a shared expert) against HF Qwen3NextForCausalLM's logits (transformers 5.15, whose
    prefill uses the chunked delta-rule form), then token-by-token decoding through the conv and
    recurrent cache states against the full forward."""
    model, ids, logits = _next_model()
    with torch.no_grad():
        ours = model(input_ids=ids, attention_mask=torch.ones_like(ids), use_cache=False).logits
        torch.testing.assert_close(ours, logits, atol=2e-4, rtol=2e-4)
        out = model(input_ids=ids[:, :5], use_cache=True)
        cache, steps = out.past_key_values, [out.logits]
        for t in range(5, ids.shape[1]):
            o = model(input_ids=ids[:, t:t + 1], past_key_values=cache, use_cache=True)
            cache = o.past_key_values
            steps.append(o.logits)
    torch.testing.assert_close(torch.cat(steps, dim=1), logits, atol=2e-4, rtol=2e-4)


def test_graph_runner_holds_no_reference_cycle():
    """A generation runner (``greedy_graphs``) refers back to its model weakly: dropping the model
    frees it and its runners by reference counting alone, never later in the cyclic garbage
    collector (which can run inside another graph's capture, where destroying graphs is not
    allowed). No graph is captured here; the runner is only created."""
    import gc
    import weakref

    cfg = QwenTritonConfig.from_hf_config(dict(model_type="qwen3", vocab_size=128, hidden_size=64,
                                               intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
                                               num_key_value_heads=2, head_dim=16, max_position_embeddings=64))
    model = QwenTritonForCausalLM(cfg)
    runner = model.greedy_graphs(1, 4, 3)
    assert runner.model is model
    gc_was_enabled = gc.isenabled()
    gc.disable()
    try:
        ref_model, ref_runner = weakref.ref(model), weakref.ref(runner)
        del model, runner
        assert ref_model() is None and ref_runner() is None
    finally:
        if gc_was_enabled:
            gc.enable()
