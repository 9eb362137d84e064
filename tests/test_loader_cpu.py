"""HF checkpoint loading from safetensors (reference: qwen_triton/loaders/hf.py:14-142).

The golden fixtures' parameters (HF names, transformers 5.15 layout) are written
as safetensors checkpoints in several on-disk forms, loaded through
``QwenTritonForCausalLM.from_pretrained_hf``, and the model's logits compared
with the golden HF logits. The report of ``load_hf_weights_into_model`` is
checked for skipped names, shape mismatches (never copied) and strict mode.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from qwen_triton import QwenTritonForCausalLM
from qwen_triton.loaders import load_hf_weights_into_model
from qwen_triton.loaders.hf import _expand_fused

GOLDEN = Path(__file__).resolve().parent / "golden"


def golden(name: str):
    d = np.load(GOLDEN / name, allow_pickle=False)
    params = {k[len("param/"):]: torch.from_numpy(d[k]) for k in d.files if k.startswith("param/")}
    cfg = {k: v for k, v in zip(d["config_keys"].tolist(), d["config_values"].tolist())}
    raw = {k: (int(v) if float(v).is_integer() and k not in ("rope_theta", "rms_norm_eps") else v) for k, v in cfg.items()}
    moe = "num_experts" in raw
    raw["model_type"] = "qwen3_moe" if moe else "qwen3"
    raw["tie_word_embeddings"] = bool(raw["tie_word_embeddings"])
    if moe:
        raw["norm_topk_prob"] = bool(raw["norm_topk_prob"])
        raw["mlp_only_layers"] = []
    return params, torch.from_numpy(d["ids"]), torch.from_numpy(d["logits"]), raw


def write_checkpoint(path: Path, params: dict, raw_cfg: dict, prefix: str = "", shards: int = 1,
                     split_experts: bool = False) -> None:
    """Write ``params`` (optionally under a wrapper prefix, optionally with the experts split per
    expert, optionally over several shards with an index file) plus config.json."""
    from safetensors.torch import save_file

    path.mkdir(parents=True, exist_ok=True)
    tensors = {}
    for k, v in params.items():
        for name, t in (_expand_fused(k, v) if split_experts else {k: v}).items():
            # a wrapper replaces the decoder's "model." (lm_head stays at the top, as in wrapped checkpoints)
            key = prefix + name[len("model."):] if prefix and name.startswith("model.") else name
            tensors[key] = t.contiguous().clone()
    keys = sorted(tensors)
    if shards == 1:
        save_file(tensors, str(path / "model.safetensors"))
    else:
        weight_map = {}
        for i in range(shards):
            fname = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
            part = {k: tensors[k] for k in keys[i::shards]}
            save_file(part, str(path / fname))
            weight_map.update({k: fname for k in part})
        (path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    (path / "config.json").write_text(json.dumps(raw_cfg))


CASES = [
    ("qwen3_tiny.npz", dict()),
    ("qwen3_tiny.npz", dict(prefix="model.language_model.", shards=3)),
    ("qwen3_tiny.npz", dict(prefix="language_model.model.")),
    ("qwen3_moe_tiny.npz", dict()),  # transformers-5 fused experts
    ("qwen3_moe_tiny.npz", dict(split_experts=True, shards=2)),  # per-expert tensors
    ("qwen3_moe_tiny.npz", dict(prefix="model.model.", split_experts=True)),
]


@pytest.mark.parametrize("name,layout", CASES)
def test_from_pretrained_hf_matches_golden_logits(tmp_path, name, layout):
    params, ids, logits, raw = golden(name)
    write_checkpoint(tmp_path / "ckpt", params, raw, **layout)
    model = QwenTritonForCausalLM.from_pretrained_hf(str(tmp_path / "ckpt"))
    with torch.no_grad():
        ours = model(input_ids=ids, attention_mask=torch.ones_like(ids), use_cache=False).logits
    torch.testing.assert_close(ours, logits, atol=1e-5, rtol=1e-4)
    report = load_hf_weights_into_model(model, tmp_path / "ckpt", strict=True)
    assert not report["missing"] and not report["mismatched"] and not report["skipped"]
    assert len(report["loaded"]) == len(dict(model.named_parameters()))


def test_report_skips_unknown_names_and_never_copies_a_wrong_shape(tmp_path):
    params, _, _, raw = golden("qwen3_tiny.npz")
    params = dict(params)
    bad = "model.layers.1.self_attn.o_proj.weight"
    params[bad] = torch.zeros(params[bad].shape[0], params[bad].shape[1] + 1)  # broadcast-incompatible shape
    params["model.layers.0.self_attn.rotary_emb.extra"] = torch.zeros(3)
    write_checkpoint(tmp_path / "ckpt", params, raw)
    model = QwenTritonForCausalLM.from_pretrained_hf(str(tmp_path / "ckpt"))
    before = model.model.layers[1].self_attn.o_proj.weight.detach().clone()
    report = load_hf_weights_into_model(model, tmp_path / "ckpt")
    assert report["skipped"] == ["model.layers.0.self_attn.rotary_emb.extra"]
    assert len(report["mismatched"]) == 1 and report["mismatched"][0].startswith(bad)
    assert report["missing"] == [bad]
    assert torch.equal(model.model.layers[1].self_attn.o_proj.weight, before)
    with pytest.raises(RuntimeError, match="unset"):
        load_hf_weights_into_model(model, tmp_path / "ckpt", strict=True)


def test_broadcastable_wrong_shape_is_reported_not_broadcast(tmp_path):
    params, _, _, raw = golden("qwen3_tiny.npz")
    params = dict(params)
    name = "model.layers.0.input_layernorm.weight"
    params[name] = torch.full((1,), 7.0)  # would broadcast over [64] under copy_
    write_checkpoint(tmp_path / "ckpt", params, raw)
    model = QwenTritonForCausalLM.from_pretrained_hf(str(tmp_path / "ckpt"))
    report = load_hf_weights_into_model(model, tmp_path / "ckpt")
    assert [m.split(" ")[0] for m in report["mismatched"]] == [name]
    assert not torch.any(model.model.layers[0].input_layernorm.weight == 7.0)


def test_missing_checkpoint_is_a_clear_error(tmp_path):
    with pytest.raises(RuntimeError, match="offline"):
        QwenTritonForCausalLM.from_pretrained_hf(str(tmp_path / "absent") + "-not-a-hub-id/x/y")
