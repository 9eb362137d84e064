"""Regenerate the golden model fixtures from HF transformers (the reference's ``ref`` backend).

Writes ``qwen3_tiny.npz``, ``qwen3_moe_tiny.npz`` and ``qwen3_next_tiny.npz``: seeded tiny-config weights
(HF parameter names, fp32), input ids, and HF's logits for them. Run from the
repo root: ``python tests/golden/make_golden.py`` (transformers 5.15 was used).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def _dump(name: str, model: torch.nn.Module, cfg: dict, ids: torch.Tensor) -> None:
    with torch.no_grad():
        logits = model(input_ids=ids, use_cache=False).logits
    arrays = {f"param/{k}": v.detach().float().numpy() for k, v in model.state_dict().items()}
    arrays["ids"] = ids.numpy()
    arrays["logits"] = logits.float().numpy()
    arrays["config_keys"] = np.array(list(cfg.keys()))
    arrays["config_values"] = np.array([float(v) for v in cfg.values()])
    np.savez_compressed(HERE / name, **arrays)
    print(name, logits.shape, float(logits.abs().max()))


def main() -> None:
    from transformers.models.qwen3.configuration_qwen3 import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3ForCausalLM
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeForCausalLM

    dense = dict(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
                 num_key_value_heads=2, head_dim=16, max_position_embeddings=64, rope_theta=10000.0,
                 rms_norm_eps=1e-6, tie_word_embeddings=0)
    torch.manual_seed(0)
    model = Qwen3ForCausalLM(Qwen3Config(**{k: (bool(v) if k == "tie_word_embeddings" else v)
                                              for k, v in dense.items()})).eval()
    with torch.no_grad():  # non-trivial norms so a dropped weight would show
        for n, p in model.named_parameters():
            if n.endswith("norm.weight"):
                p.uniform_(0.5, 1.5)
    ids = torch.randint(0, 128, (2, 8), generator=torch.Generator().manual_seed(1))
    _dump("qwen3_tiny.npz", model, dense, ids)

    moe = dict(vocab_size=128, hidden_size=64, intermediate_size=96, num_hidden_layers=2, num_attention_heads=4,
               num_key_value_heads=2, head_dim=16, max_position_embeddings=64, rope_theta=10000.0, rms_norm_eps=1e-6,
               decoder_sparse_step=1, moe_intermediate_size=32, num_experts=4, num_experts_per_tok=2,
               norm_topk_prob=1, tie_word_embeddings=0)
    torch.manual_seed(0)
    hf_cfg = Qwen3MoeConfig(**{k: (bool(v) if k in ("norm_topk_prob", "tie_word_embeddings") else v)
                               for k, v in moe.items()}, mlp_only_layers=[])
    model = Qwen3MoeForCausalLM(hf_cfg).eval()
    with torch.no_grad():
        for i, (n, p) in enumerate(model.named_parameters()):
            if "experts" in n or n.endswith("gate.weight"):
                p.normal_(0.0, 0.2, generator=torch.Generator().manual_seed(i))
    ids = torch.randint(0, 128, (2, 6), generator=torch.Generator().manual_seed(2))
    _dump("qwen3_moe_tiny.npz", model, moe, ids)

    # Qwen3-Next: linear-attention (gated delta rule) and gated full-attention layers, partial
    # rotary, (1 + w) norms, MoE with a shared expert
    from transformers.models.qwen3_next.configuration_qwen3_next import Qwen3NextConfig
    from transformers.models.qwen3_next.modeling_qwen3_next import Qwen3NextForCausalLM

    nxt = dict(vocab_size=128, hidden_size=64, intermediate_size=96, num_hidden_layers=4, num_attention_heads=4,
               num_key_value_heads=2, head_dim=16, max_position_embeddings=64, rms_norm_eps=1e-6,
               tie_word_embeddings=0, linear_conv_kernel_dim=4, linear_key_head_dim=16, linear_value_head_dim=8,
               linear_num_key_heads=2, linear_num_value_heads=4, decoder_sparse_step=1, moe_intermediate_size=32,
               shared_expert_intermediate_size=48, num_experts_per_tok=2, num_experts=4, norm_topk_prob=1,
               full_attention_interval=2, rope_theta=10000.0, partial_rotary_factor=0.25)
    torch.manual_seed(0)
    hf_cfg = Qwen3NextConfig(**{k: (bool(v) if k in ("norm_topk_prob", "tie_word_embeddings") else v)
                                for k, v in nxt.items() if k not in ("full_attention_interval", "rope_theta",
                                                                     "partial_rotary_factor")},
                             layer_types=["linear_attention", "full_attention"] * 2,
                             rope_parameters={"rope_type": "default", "rope_theta": 10000.0,
                                              "partial_rotary_factor": 0.25},
                             mlp_only_layers=[])
    model = Qwen3NextForCausalLM(hf_cfg).eval()
    with torch.no_grad():  # non-trivial norms, decays and gates so a dropped term would show
        for i, (n, p) in enumerate(model.named_parameters()):
            gen = torch.Generator().manual_seed(100 + i)
            if n.endswith("norm.weight"):
                p.copy_(torch.rand(p.shape, generator=gen) * 0.5 - 0.25)
            elif n.endswith("A_log"):
                p.copy_(torch.rand(p.shape, generator=gen) * 2.0 - 1.0)
            elif n.endswith("dt_bias"):
                p.copy_(torch.rand(p.shape, generator=gen))
            else:
                p.copy_(torch.randn(p.shape, generator=gen) * 0.1)
    ids = torch.randint(0, 128, (2, 9), generator=torch.Generator().manual_seed(3))
    _dump("qwen3_next_tiny.npz", model, nxt, ids)


if __name__ == "__main__":
    main()
