"""Offline HF checkpoint loading (reference: qwen_triton/loaders/hf.py:14-142).

A checkpoint is a local directory (or a snapshot already in the local HF cache:
there is no network here) holding ``config.json`` and ``*.safetensors`` shards,
listed by ``model.safetensors.index.json`` when present.

Checkpoint names are matched to the model's parameters and persistent buffers
after removing the wrappers multimodal and nested checkpoints put around a
causal LM (``language_model.``, ``model.language_model.``,
``model.language_model.model.``, ``model.model.``) and trying the name with and
without a leading ``model.`` (reference :80-104). Qwen3-MoE checkpoints written
by transformers >= 5 store each layer's experts fused (``mlp.experts.gate_up_proj``
[E, 2I, H] with the gate half first, ``mlp.experts.down_proj`` [E, H, I]); they
are split into this model's per-expert ``experts.{e}.{gate,up,down}_proj.weight``
before matching. Both layouts load.

``load_hf_weights_into_model`` keeps the reference's contract (:107-142):
tensors of a matching name and shape are copied (cast to the target's dtype and
device); names with no target are reported as ``skipped``, shape disagreements
as ``mismatched`` (never copied); targets left unset are ``missing``, an error
only with ``strict=True``.
"""
from __future__ import annotations

import json
import re
from pathlib import Path
from typing import Iterator

import torch

_FUSED_RE = re.compile(r"^(.*\.mlp\.experts)\.(gate_up_proj|down_proj)$")
# wrappers around a causal LM's own names, longest first
_WRAPPERS = ("model.language_model.model.", "model.language_model.", "language_model.", "model.model.")


def ensure_local_model_path(model_id_or_path: str, include_weights: bool = True) -> Path:
    """The checkpoint directory: ``model_id_or_path`` itself when it exists, else a snapshot of that
    hub id already in the local HF cache (nothing is downloaded)."""
    path = Path(model_id_or_path)
    if path.exists():
        return path
    patterns = ["config.json", "generation_config.json", "tokenizer*", "*.model", "vocab.json", "merges.txt"]
    if include_weights:
        patterns += ["*.safetensors", "*.safetensors.index.json"]
    try:
        from huggingface_hub import snapshot_download

        return Path(snapshot_download(repo_id=model_id_or_path, allow_patterns=patterns, local_files_only=True))
    except Exception as exc:
        raise RuntimeError(f"{model_id_or_path!r} is neither a local path nor a snapshot in the local HF cache "
                           "(checkpoints must be available offline)") from exc


def load_config_dict(model_id_or_path: str) -> dict:
    path = ensure_local_model_path(model_id_or_path, include_weights=False)
    cfg = path / "config.json" if path.is_dir() else path
    return json.loads(cfg.read_text(encoding="utf-8"))


def _shards(snapshot_path: Path) -> list[Path]:
    index = snapshot_path / "model.safetensors.index.json"
    if index.exists():
        weight_map = json.loads(index.read_text(encoding="utf-8"))["weight_map"]
        return sorted({snapshot_path / f for f in weight_map.values()})
    files = sorted(snapshot_path.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no safetensors files under {snapshot_path}")
    return files


def iter_safetensor_tensors(snapshot_path: Path) -> Iterator[tuple[str, torch.Tensor]]:
    """(name, tensor) of every tensor in the checkpoint, shard by shard, on the CPU."""
    from safetensors import safe_open

    for shard in _shards(Path(snapshot_path)):
        with safe_open(str(shard), framework="pt", device="cpu") as f:
            for key in f.keys():
                yield key, f.get_tensor(key)


def _expand_fused(name: str, tensor: torch.Tensor) -> dict[str, torch.Tensor]:
    """A fused expert tensor as per-expert weights; any other tensor unchanged."""
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


def _target_name(key: str, targets) -> str | None:
    """The model name a checkpoint name stands for, or None."""
    forms = [key]
    for wrapper in _WRAPPERS:
        if key.startswith(wrapper):
            inner = key[len(wrapper):]
            forms += [inner, "model." + inner]
    forms.append(key[len("model."):] if key.startswith("model.") else "model." + key)
    return next((f for f in forms if f in targets), None)


def load_hf_weights_into_model(model: torch.nn.Module, snapshot_path, strict: bool = False) -> dict[str, list[str]]:
    """Copy the checkpoint's tensors into ``model``; returns the report
    ``{"loaded", "missing", "skipped", "mismatched"}`` (lists of names)."""
    targets = dict(model.named_parameters())
    persistent = set(model.state_dict().keys())
    targets.update({n: b for n, b in model.named_buffers() if n in persistent})
    loaded: set[str] = set()
    skipped: list[str] = []
    mismatched: list[str] = []
    with torch.no_grad():
        for key, stored in iter_safetensor_tensors(Path(snapshot_path)):
            fused = _FUSED_RE.match(key) is not None
            for name, tensor in _expand_fused(key, stored).items():
                label = f"{key}[{name}]" if fused else key
                target_name = _target_name(name, targets)
                if target_name is None:
                    skipped.append(label)
                    continue
                target = targets[target_name]
                if tuple(target.shape) != tuple(tensor.shape):
                    mismatched.append(f"{label} -> {target_name}: {tuple(tensor.shape)} != {tuple(target.shape)}")
                    continue
                target.copy_(tensor.to(device=target.device, dtype=target.dtype))
                loaded.add(target_name)
    missing = sorted(set(targets) - loaded)
    if strict and missing:
        raise RuntimeError(f"checkpoint leaves {len(missing)} parameters unset, e.g. {missing[:20]}")
    return {"loaded": sorted(loaded), "missing": missing, "skipped": skipped, "mismatched": mismatched}
