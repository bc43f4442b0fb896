"""Device-resident greedy decode steps, optionally replayed from a HIP graph.

The reference's ``ModelRunner.execute`` (src/llmserve/model_runner.py:40-87) rebuilds the
attention metadata on the host for every step, runs the model, copies the logits to the host
and samples there (sampling.py:169-170). For a batch of sequences that are all decoding, every
piece of that state can live on the GPU: the block tables (sized up front for the longest
context the run will reach), the context lengths (advanced on the device by the greedy kernel)
and the last token of each sequence. ``DecodeRunner.step`` is then one fixed sequence of
kernels with no host round trip, so it is captured once into a HIP graph and replayed
(``torch.cuda.CUDAGraph``); each replay decodes one token per sequence.

Graph capture records no memset nodes: every buffer the step writes is written by a kernel.
"""

from __future__ import annotations

import torch

from llmserve.kernels import load_fused_ops
from llmserve.kv_cache import KVCache
from llmserve.transformer import QuantCausalLM


class DecodeRunner:
    """Greedy decode of a fixed batch of sequences.

    ``ids`` [B]: the last token of each sequence (the one to decode now); ``context_lens`` [B]:
    tokens of each sequence including that one; ``block_tables`` [B, max_blocks]: physical
    blocks of each sequence, wide enough for every position the run will reach. The three are
    copied into device buffers owned by the runner; ``step`` / ``replay`` update them in place
    (ids <- next token, context_lens += 1)."""

    def __init__(self, model: QuantCausalLM, cache: KVCache, ids: torch.Tensor,
                 context_lens: torch.Tensor, block_tables: torch.Tensor) -> None:
        if cache.kv_dtype != "int8":
            raise ValueError("DecodeRunner runs the int8 KV cache")
        dev = model.embed.device
        B = ids.numel()
        if context_lens.numel() != B or block_tables.shape[0] != B:
            raise ValueError("one context length and one block-table row per sequence")
        self.model, self.cache = model, cache
        self.block_size = cache.block_size
        self.ids = ids.to(device=dev, dtype=torch.long).contiguous().clone()
        self.context_lens = context_lens.to(device=dev, dtype=torch.long).contiguous().clone()
        self.block_tables = block_tables.to(device=dev, dtype=torch.long).contiguous().clone()
        self.max_context = self.block_tables.shape[1] * self.block_size
        self.logits: torch.Tensor | None = None
        self.graph: torch.cuda.CUDAGraph | None = None

    def forward_logits(self) -> torch.Tensor:
        """Logits [B, V] of the current tokens; writes their K/V but does not advance."""
        m = self.model
        h = m.forward_decode(self.ids, self.context_lens, self.block_tables, self.cache.layers,
                             self.block_size)
        B = self.ids.numel()
        return m.compute_logits(h, B if m._lm_frag(B) else None)

    def _step(self) -> None:
        self.logits = self.forward_logits()
        nxt = load_fused_ops().argmax_advance(self.logits, self.context_lens)
        self.ids.copy_(nxt)

    def step(self) -> torch.Tensor:
        """Decode one token per sequence eagerly; returns the ids buffer (the new tokens)."""
        self._step()
        return self.ids

    def capture(self, keep_state: bool = True) -> None:
        """Record one step into a HIP graph. One eager step runs first, on a side stream, so
        that kernel attributes, library handles and workspaces are set up outside the graph;
        with ``keep_state`` the ids, context lengths and caches are restored after it, else
        that step counts as a decoded token."""
        saved = self.snapshot() if keep_state else None
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self._step()
        torch.cuda.current_stream().wait_stream(s)
        if saved is not None:
            self.restore(saved)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._step()
        self.graph = g

    def snapshot(self):
        """Copies of the state a step changes (ids, context lengths, every cache tensor)."""
        return (self.ids.clone(), self.context_lens.clone(),
                [(k.data.clone(), k.scale.clone(), v.data.clone(), v.scale.clone())
                 for k, v in self.cache.layers])

    def restore(self, saved) -> None:
        ids, ctx, layers = saved
        self.ids.copy_(ids)
        self.context_lens.copy_(ctx)
        for (k, v), (kd, ks, vd, vs) in zip(self.cache.layers, layers, strict=True):
            k.data.copy_(kd)
            k.scale.copy_(ks)
            v.data.copy_(vd)
            v.scale.copy_(vs)

    def replay(self) -> torch.Tensor:
        """One graph replay = one decode step; returns the ids buffer."""
        if self.graph is None:
            raise RuntimeError("capture() first")
        self.graph.replay()
        return self.ids
