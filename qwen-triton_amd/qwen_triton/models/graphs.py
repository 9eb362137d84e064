"""Captured greedy generation: the prefill and the decode step as two HIP graphs, kept for reuse.

Reference: the eager loop of qwen_triton/models/core.py:378-410 (``greedy_generate``), which
re-runs the Python of every layer for each token. A serving loop that generates for prompts of
one shape many times replays these graphs instead:

* the prefill graph runs the forward over the prompt buffer into a preallocated cache, picks
  the first token (top-1 on the library kernel, ties to the lowest index as argmax) and resets
  the device-side decode state (cache position, valid lengths, next output column);
* the step graph decodes one token from that device state and advances it.

Both are captured on first use. Each replay overwrites the same buffers (cache, tokens), so a
runner serves one call at a time; the graphs hold the parameters' storage addresses, so a model
whose parameters are replaced (not updated in place) gets new runners (the owner keys them on
those addresses).
"""
from __future__ import annotations

import torch

from qwen_triton.modules.cache import StaticDecode


def _pick(logits: torch.Tensor) -> torch.Tensor:
    from qwen_triton.kernels.moe_routing import _native_topk

    return _native_topk(logits[:, -1], 1)[1]


class GreedyGraphs:
    def __init__(self, model, batch: int, prompt: int, max_new: int, dtype: torch.dtype, device) -> None:
        if max_new < 2:
            raise ValueError("graph-captured generation needs at least two new tokens")
        self.model = model
        self.batch, self.prompt, self.max_new = batch, prompt, max_new
        self.cache = model.new_cache(batch, prompt + max_new, dtype, device)
        self.prompt_ids = torch.zeros((batch, prompt), dtype=torch.long, device=device)
        self.tokens = torch.zeros((batch, max_new), dtype=torch.long, device=device)
        self.ids = torch.zeros((batch, 1), dtype=torch.long, device=device)
        self.col = torch.ones((1, 1), dtype=torch.long, device=device)
        self.static = StaticDecode(positions=torch.full((1,), prompt, dtype=torch.long, device=device),
                                   seqlens=torch.full((batch,), prompt + 1, dtype=torch.int32, device=device))
        self.prefill_graph: torch.cuda.CUDAGraph | None = None
        self.step_graph: torch.cuda.CUDAGraph | None = None

    def _prefill_body(self) -> None:
        cache = self.cache
        cache.static = None
        cache.attention_lengths = [0] * cache.num_layers  # prefill from position 0
        logits = self.model(input_ids=self.prompt_ids, past_key_values=cache, use_cache=True, logits_to_keep=1).logits
        first = _pick(logits)
        self.tokens[:, :1].copy_(first)
        self.ids.copy_(first)
        self.col.fill_(1)
        self.static.positions.fill_(self.prompt)
        self.static.seqlens.fill_(self.prompt + 1)

    def _step_body(self) -> None:
        self.cache.static = self.static
        try:
            logits = self.model(input_ids=self.ids, past_key_values=self.cache, use_cache=True,
                                logits_to_keep=1).logits
        finally:
            self.cache.static = None
        nxt = _pick(logits)
        self.ids.copy_(nxt)
        self.tokens.scatter_(1, self.col.expand(self.batch, 1), nxt)
        self.col.add_(1)
        self.static.positions.add_(1)
        self.static.seqlens.add_(1)

    def _capture(self) -> None:
        dev = self.prompt_ids.device
        # eager warm-up on a side stream (builds the host-side plans, rotary tables and pools)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            self._prefill_body()
            self._step_body()
        torch.cuda.current_stream(dev).wait_stream(side)
        prefill, step = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        with torch.cuda.graph(prefill):
            self._prefill_body()
        with torch.cuda.graph(step):
            self._step_body()
        self.prefill_graph, self.step_graph = prefill, step

    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Replay the prefill for ``input_ids`` [batch, prompt]; returns the first new tokens [batch, 1]
        (a view of the runner's buffer)."""
        if tuple(input_ids.shape) != (self.batch, self.prompt):
            raise ValueError(f"runner shape {(self.batch, self.prompt)} != input {tuple(input_ids.shape)}")
        self.prompt_ids.copy_(input_ids)
        if self.prefill_graph is None:
            self._capture()
        self.prefill_graph.replay()
        return self.tokens[:, :1]

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Greedy tokens for ``input_ids``: [batch, prompt + max_new] (prompt, then the new tokens)."""
        self.prefill(input_ids)
        for _ in range(self.max_new - 1):
            self.step_graph.replay()
        return torch.cat((input_ids, self.tokens), dim=-1)
