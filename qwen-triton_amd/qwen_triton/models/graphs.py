"""Captured greedy generation: the prefill and the decode step as two HIP graphs, kept for reuse.

Reference: the eager loop of qwen_triton/models/core.py:378-410 (``greedy_generate``), which
re-runs the Python of every layer for each token. A serving loop that generates for prompts of
one shape many times replays these graphs instead:

* the prefill graph runs the forward over the prompt buffer into a preallocated cache, picks
  the first token and resets the device-side decode state (cache position, valid lengths, next
  output column);
* the step graph decodes one token from that device state and advances it.

The pick is torch.argmax's (NaN largest, ties to the lowest index); it and the state updates
are two library launches (``qh_greedy_step``), or for more than 64 rows a top-1 kernel and
torch ops on the same buffers.

Both are captured on first use. Each replay overwrites the same buffers (cache, tokens), so a
runner serves one call at a time. The graphs hold the addresses of the parameters and of tensors
derived from them (norm-folded weights, rotary tables): the owner keys runners on the parameters'
storage and version counters, so replaced or in-place-updated parameters get new runners, and a
runner holds references to the derived tensors its graphs read, so that a rebuilt fold or a
regrown rotary table never frees memory a graph still reads.
"""
from __future__ import annotations

import gc
import weakref

import torch

from qwen_triton import _native
from qwen_triton.modules.cache import StaticDecode


def _pick(logits: torch.Tensor) -> torch.Tensor:
    from qwen_triton.kernels.moe_routing import _native_topk

    return _native_topk(logits[:, -1], 1)[1]


_GREEDY_MAX_ROWS = 64  # rows qh_greedy_step serves
_GREEDY_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _greedy_step_ok(batch: int, vocab: int, dtype: torch.dtype) -> bool:
    return batch <= _GREEDY_MAX_ROWS and dtype in _GREEDY_DTYPES \
        and (vocab * torch.tensor([], dtype=dtype).element_size()) % 16 == 0


class GreedyGraphs:
    def __init__(self, model, batch: int, prompt: int, max_new: int, dtype: torch.dtype, device) -> None:
        if max_new < 2:
            raise ValueError("graph-captured generation needs at least two new tokens")
        # The owner model keeps its runners; a weak reference back avoids a reference cycle, which
        # only the cyclic garbage collector would free, at an arbitrary later allocation (possibly
        # inside another graph's capture, where destroying graphs is not allowed).
        self._model = weakref.ref(model)
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
        self._derived: list[torch.Tensor] = []
        # the pick and the step's bookkeeping in two library launches (qh_greedy_step) when the
        # shape allows; otherwise top-1 and torch ops on the same buffers
        vocab = model.config.vocab_size
        self.greedy_ws = None
        if _greedy_step_ok(batch, vocab, dtype):
            self.greedy_ws = _native.workspace(_native.call("qh_greedy_step_workspace", batch, vocab), device)

    @property
    def model(self):
        m = self._model()
        if m is None:
            raise RuntimeError("the model of this generation runner no longer exists")
        return m

    def _greedy(self, logits: torch.Tensor) -> None:
        last = logits[:, -1]
        if last.stride(-1) != 1 or last.data_ptr() % 16 or (last.stride(0) * last.element_size()) % 16:
            last = last.contiguous()
        _native.call("qh_greedy_step", last.data_ptr(), last.stride(0), self.batch, last.shape[-1],
                     self.ids.data_ptr(), self.tokens.data_ptr(), self.tokens.stride(0), self.tokens.shape[1],
                     self.col.data_ptr(), self.static.positions.data_ptr(), self.static.seqlens.data_ptr(),
                     self.greedy_ws.data_ptr(), self.greedy_ws.numel(), _native.dtype_code(last.dtype),
                     _native.stream(last.device))

    def _prefill_body(self) -> None:
        cache = self.cache
        cache.static = None
        cache.attention_lengths = [0] * cache.num_layers  # prefill from position 0
        logits = self.model(input_ids=self.prompt_ids, past_key_values=cache, use_cache=True, logits_to_keep=1).logits
        if self.greedy_ws is not None and logits.dtype in _GREEDY_DTYPES:
            # the step kernel stores the first token at column 0 and leaves col = 1,
            # position = prompt, lengths = prompt + 1
            self.col.fill_(0)
            self.static.positions.fill_(self.prompt - 1)
            self.static.seqlens.fill_(self.prompt)
            self._greedy(logits)
            return
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
        if self.greedy_ws is not None and logits.dtype in _GREEDY_DTYPES:
            self._greedy(logits)
            return
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
        # no cyclic garbage collection while capturing: an unreachable object that owns device
        # resources (another graph, say) must not be destroyed inside a capture
        gc_was_enabled = gc.isenabled()
        gc.collect()
        gc.disable()
        try:
            with torch.cuda.graph(prefill):
                self._prefill_body()
            with torch.cuda.graph(step):
                self._step_body()
        finally:
            if gc_was_enabled:
                gc.enable()
        self.prefill_graph, self.step_graph = prefill, step
        self._derived = self._derived_tensors()

    def _derived_tensors(self) -> list[torch.Tensor]:
        """Tensors the captured graphs read that the model keeps outside its parameters: the
        norm-folded weights and the rotary tables (held here so they outlive a rebuild)."""
        from qwen_triton.kernels.matmul import folded_weight_tensors
        from qwen_triton.modules.rotary import QwenRotaryEmbedding

        held = folded_weight_tensors(self.model)
        for mod in self.model.modules():
            if isinstance(mod, QwenRotaryEmbedding):
                held.extend(mod._tables.values())
        return held

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
