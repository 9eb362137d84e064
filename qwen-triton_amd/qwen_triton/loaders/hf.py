"""Offline HF checkpoint loading (reference: qwen_triton/loaders/hf.py:14-142).

Only local directories are supported (this stack runs without network access):
``config.json`` plus ``*.safetensors`` shards. Parameter names of
``QwenTritonForCausalLM`` equal HF's Qwen3 names; Qwen3-MoE checkpoints written
by transformers >= 5 store experts fused (``mlp.experts.gate_up_proj`` [E, 2I, H]
with the gate half first, ``mlp.experts.down_proj`` [E, H, I]) and are split
into the per-expert ``experts.{i}.{gate,up,down}_proj.weight`` layout here.
"""
from __future__ import annotations

import json
import re
from pathlib import Path

import torch

_FUSED_RE = re.compile(r"^(.*\.mlp\.experts)\.(gate_up_proj|down_proj)$")


def ensure_local_model_path(model_id: str, include_weights: bool = True) -> Path:
    path = Path(model_id)
    if not path.is_dir():
        raise RuntimeError(f"{model_id!r} is not a local directory; checkpoints must be available offline")
    if include_weights and not any(path.glob("*.safetensors")):
        raise RuntimeError(f"no *.safetensors files under {path}")
    return path


def load_config_dict(model_id: str) -> dict:
    path = ensure_local_model_path(model_id, include_weights=False)
    return json.loads((path / "config.json").read_text())


def _expand_fused(name: str, tensor: torch.Tensor) -> dict[str, torch.Tensor]:
    m = _FUSED_RE.match(name)
    if m is None:
        return {name: tensor}
    prefix, kind = m.groups()
    out = {}
    if kind == "gate_up_proj":
        inter = tensor.shape[1] // 2
        for e in range(tensor.shape[0]):
            out[f"{prefix}.{e}.gate_proj.weight"] = tensor[e, :inter]
            out[f"{prefix}.{e}.up_proj.weight"] = tensor[e, inter:]
    else:
        for e in range(tensor.shape[0]):
            out[f"{prefix}.{e}.down_proj.weight"] = tensor[e]
    return out


def load_hf_weights_into_model(model: torch.nn.Module, snapshot_path: str | Path) -> None:
    from safetensors import safe_open

    params = dict(model.named_parameters())
    loaded = set()
    for shard in sorted(Path(snapshot_path).glob("*.safetensors")):
        with safe_open(str(shard), framework="pt") as f:
            for key in f.keys():
                for name, tensor in _expand_fused(key, f.get_tensor(key)).items():
                    if name in params:
                        with torch.no_grad():
                            params[name].copy_(tensor.to(params[name].dtype))
                        loaded.add(name)
    missing = [n for n in params if n not in loaded and not (n == "lm_head.weight" and model.config.tie_word_embeddings)]
    if missing:
        raise RuntimeError(f"checkpoint is missing {len(missing)} parameters, e.g. {missing[:3]}")
