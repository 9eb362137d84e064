"""CPU restatement of the ``ref`` backend: HF-semantics Qwen3 / Qwen3-MoE (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this module. It evaluates the model functionally from a parameter
dict whose names are those of ``QwenTritonForCausalLM`` (= HF Qwen3 names),
following transformers 5.15 ``models/qwen3/modeling_qwen3.py`` (RMSNorm :50-64,
MLP :70-83, RoPE :86-170, eager attention :185-208, layer :283-324, causal LM
with ``logits_to_keep`` :431-507) and ``models/qwen3_moe/modeling_qwen3_moe.py``
(experts :210-246, router :249-267), as exercised by the reference's ``ref``
path (qwen_triton/models/core.py:274-281, :335-346) and the reference model's
own composition (qwen_triton/models/core.py:95-247).

Pinned by ``tests/test_oracle.py`` against HF ``Qwen3ForCausalLM`` /
``Qwen3MoeForCausalLM`` on shared weights, the committed golden logits under
``tests/golden/`` and the cached-decode == full-forward invariant of the
reference's tests/test_model_parity.py:42-80.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import ops


@dataclass
class ModelSpec:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    tie_word_embeddings: bool = False
    num_experts: int = 0
    num_experts_per_tok: int = 0
    moe_intermediate_size: int = 0
    norm_topk_prob: bool = True
    decoder_sparse_step: int = 1
    mlp_only_layers: list = field(default_factory=list)

    @classmethod
    def from_config(cls, cfg) -> "ModelSpec":
        return cls(**{k: getattr(cfg, k) for k in cls.__dataclass_fields__ if hasattr(cfg, k)})

    def layer_is_moe(self, i: int) -> bool:
        return self.num_experts > 0 and i not in self.mlp_only_layers and (i + 1) % self.decoder_sparse_step == 0


class OracleQwen:
    """Functional Qwen3 causal LM on CPU tensors of ``dtype`` with an optional KV cache."""

    def __init__(self, spec: ModelSpec, params: dict, dtype=torch.float32) -> None:
        self.spec = spec
        self.dtype = dtype
        self.p = {k: v.detach().to("cpu", dtype) for k, v in params.items()}
        if spec.tie_word_embeddings or "lm_head.weight" not in self.p:
            self.p["lm_head.weight"] = self.p["model.embed_tokens.weight"]

    # HF Qwen3RMSNorm: normalise in fp32, cast back, then scale by the weight.
    def _norm(self, x, w):
        xf = x.to(torch.float32)
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.spec.rms_norm_eps)
        return w * xf.to(x.dtype)

    def _rope(self, x, cos, sin):
        half = x.shape[-1] // 2
        rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
        return x * cos[:, None] + rot * sin[:, None]

    def _mlp(self, pre, x):
        p = self.p
        g = x @ p[pre + "gate_proj.weight"].T
        return (torch.nn.functional.silu(g) * (x @ p[pre + "up_proj.weight"].T)) @ p[pre + "down_proj.weight"].T

    def _moe(self, pre, x):
        s, p = self.spec, self.p
        B, S, H = x.shape
        flat = x.reshape(-1, H)
        logits = flat @ p[pre + "gate.weight"].T
        probs = torch.softmax(logits.to(torch.float32), dim=-1)
        w, e = ops.topk(probs, s.num_experts_per_tok)
        if s.norm_topk_prob:
            w = w / w.sum(-1, keepdim=True)
        w = w.to(x.dtype)
        out = torch.zeros_like(flat)
        for ex in range(s.num_experts):
            tok, slot = torch.where(e == ex)
            if tok.numel() == 0:
                continue
            h = self._mlp(f"{pre}experts.{ex}.", flat[tok]) * w[tok, slot, None]
            out.index_add_(0, tok, h.to(flat.dtype))
        return out.view(B, S, H)

    def new_cache(self):
        return {"k": [None] * self.spec.num_hidden_layers, "v": [None] * self.spec.num_hidden_layers, "len": 0}

    def forward(self, input_ids: torch.Tensor, cache: dict | None = None, logits_to_keep: int = 0):
        s, p = self.spec, self.p
        ids = input_ids.cpu().long()
        B, S = ids.shape
        past = 0 if cache is None else cache["len"]
        pos = torch.arange(past, past + S)
        cos, sin = ops.rotary_tables(pos, s.head_dim, s.rope_theta, torch.float32)
        cos, sin = cos.to(self.dtype), sin.to(self.dtype)
        x = p["model.embed_tokens.weight"][ids]
        groups = s.num_attention_heads // s.num_key_value_heads
        scale = s.head_dim ** -0.5
        for i in range(s.num_hidden_layers):
            pre = f"model.layers.{i}."
            h = self._norm(x, p[pre + "input_layernorm.weight"])
            q = (h @ p[pre + "self_attn.q_proj.weight"].T).view(B, S, -1, s.head_dim)
            k = (h @ p[pre + "self_attn.k_proj.weight"].T).view(B, S, -1, s.head_dim)
            v = (h @ p[pre + "self_attn.v_proj.weight"].T).view(B, S, -1, s.head_dim).transpose(1, 2)
            q = self._norm(q, p[pre + "self_attn.q_norm.weight"]).transpose(1, 2)
            k = self._norm(k, p[pre + "self_attn.k_norm.weight"]).transpose(1, 2)
            q, k = self._rope(q, cos, sin), self._rope(k, cos, sin)
            if cache is not None:
                if cache["k"][i] is not None:
                    k = torch.cat((cache["k"][i], k), dim=2)
                    v = torch.cat((cache["v"][i], v), dim=2)
                cache["k"][i], cache["v"][i] = k, v
            kv = k.shape[2]
            ke, ve = k.repeat_interleave(groups, 1), v.repeat_interleave(groups, 1)
            scores = (q @ ke.transpose(-1, -2)) * scale
            allowed = torch.arange(kv)[None, :] <= (torch.arange(S) + past)[:, None]
            scores = scores.masked_fill(~allowed, torch.finfo(scores.dtype).min)
            attn = torch.softmax(scores.to(torch.float32), dim=-1).to(q.dtype) @ ve
            attn = attn.transpose(1, 2).reshape(B, S, -1)
            x = x + attn @ p[pre + "self_attn.o_proj.weight"].T
            h = self._norm(x, p[pre + "post_attention_layernorm.weight"])
            x = x + (self._moe(pre + "mlp.", h) if s.layer_is_moe(i) else self._mlp(pre + "mlp.", h))
        if cache is not None:
            cache["len"] = past + S
        x = self._norm(x, p["model.norm.weight"])
        if logits_to_keep > 0:
            x = x[:, -logits_to_keep:]
        return x @ p["lm_head.weight"].T

    def greedy_generate(self, input_ids: torch.Tensor, max_new_tokens: int) -> torch.Tensor:
        cache = self.new_cache()
        ids = input_ids.cpu().long()
        step = ids
        for _ in range(max_new_tokens):
            logits = self.forward(step, cache, logits_to_keep=1)
            nxt = logits[:, -1].argmax(-1, keepdim=True)
            ids = torch.cat((ids, nxt), dim=-1)
            step = nxt
        return ids
