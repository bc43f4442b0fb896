"""Model execution for a scheduled batch, and device-resident greedy decode steps.

``ModelRunner`` keeps the reference's interface (src/llmserve/model_runner.py:14-87): it turns
one scheduler step (``sched.scheduled``: per sequence its token ids, computed-token count, new
token count and block table; ``sched.block_copies``) into one forward pass and returns the
requested logits rows on the host. A step whose sequences all decode one token over an int8
cache runs the fused decode step (``QuantCausalLM.forward_decode``: the KV write fused into the
post-qkv kernel, attention merges writing the next linear's input); any other batch (prompt
chunks, mixed batches, fp32 caches) runs the ragged forward with device-built attention
metadata and one paged-attention launch per layer over all tokens.

``DecodeRunner`` goes further for a fixed batch that only decodes: the block tables (sized up
front for the longest context the run will reach), the context lengths (advanced on the device
by the greedy kernel) and the last token of each sequence live on the GPU, so a step is one
fixed sequence of kernels with no host round trip, captured once into a HIP graph and replayed
(``torch.cuda.CUDAGraph``); each replay decodes one token per sequence. Graph capture records
no memset nodes: every buffer the step writes is written by a kernel.
"""

from __future__ import annotations

import numpy as np
import torch

from .attention import AttentionMetadata, QuantizedKV, _model_placement, resolve_backend
from .kernels import load_fused_ops
from .kv_cache import KVCache
from .transformer import QuantCausalLM


class ModelRunner:
    """One forward pass per scheduled batch (reference model_runner.py:14-87)."""

    # decode-only steps over an int8 cache take the fused decode step of QuantCausalLM
    fused_decode = True

    def __init__(self, model, kv_cache: KVCache, attention_backend: str = "auto") -> None:
        self.model = model
        self.cache = kv_cache
        self.block_size = kv_cache.block_size
        self.device, dtype = _model_placement(model)
        if attention_backend == "auto" and dtype != torch.float32:
            attention_backend = "torch"  # the native kernels serve fp32 models
        self.attention_backend = resolve_backend(attention_backend, str(self.device))

    def copy_blocks(self, copies: list[tuple[int, int]]) -> None:
        """Copies whole blocks (src, dst) in every layer's K and V cache (copy-on-write)."""
        if not copies:
            return
        bs = self.block_size
        pairs = np.asarray(copies, dtype=np.int64).reshape(-1, 2)
        offs = np.arange(bs)
        src = torch.from_numpy((pairs[:, :1] * bs + offs).reshape(-1))
        dst = torch.from_numpy((pairs[:, 1:] * bs + offs).reshape(-1))
        for pair in self.cache.layers:
            for c in pair:
                if isinstance(c, QuantizedKV):
                    c.copy_rows(dst, src)
                else:
                    c.index_copy_(0, dst.to(c.device), c.index_select(0, src.to(c.device)))

    def _check_tables(self, tables, ctx_lens) -> None:
        """Every block a context uses must lie inside the cache. The reference's cache write
        (``index_copy_``, attention.py:159-162) raises on a slot past the cache; the native
        write kernels skip such slots instead, so the host checks the tables it already holds
        (no device synchronization) and raises the same way."""
        if not tables:
            return
        bs = self.block_size
        slots = self.cache.num_blocks * bs
        for t, c in zip(tables, ctx_lens):
            used = np.asarray(t[: -(-c // bs)], dtype=np.int64)
            if used.size == 0:
                continue  # a table too short is reported by the metadata build
            lo, hi = int(used.min()), int(used.max())
            if lo < 0 or (hi + 1) * bs > slots:
                bad = lo if lo < 0 else hi
                raise IndexError(f"index_copy_(): block {bad} (slots {bad * bs}..{bad * bs + bs - 1})"
                                 f" is out of bounds for a cache of {slots} slots")

    @staticmethod
    def _check_ids(ids, vocab: int) -> None:
        """Token ids must index the embedding. The reference's ``nn.Embedding`` raises on one
        outside [0, vocab); the native gather writes a NaN row instead, so the host checks the
        ids it already holds and raises as torch does."""
        if ids and (min(ids) < 0 or max(ids) >= vocab):
            raise IndexError("index out of range in self")

    def _decode_step_ok(self, q_lens: list[int], logit_rows: list[int]) -> bool:
        m = self.model
        return (self.fused_decode and isinstance(m, QuantCausalLM)
                and self.cache.kv_dtype == "int8" and self.device.type == "cuda"
                and load_fused_ops() is not None and all(n == 1 for n in q_lens)
                and len(logit_rows) == len(set(logit_rows)))

    @torch.inference_mode()
    def execute(
        self,
        sched,
        sample_rows: list[int],
        num_logits: dict[int, int] | None = None,
    ) -> torch.Tensor:
        """Runs the model on ``sched``; returns (on the host) the logits of the last new token
        of each ``sched.scheduled[i]`` for i in ``sample_rows`` (the last ``num_logits[i]``
        positions when given: speculative verification), in order."""
        self.copy_blocks(getattr(sched, "block_copies", None) or [])
        ids: list[int] = []
        pos: list[int] = []
        q_lens, ctx_lens, tables, last = [], [], [], []
        for item in sched.scheduled:
            seq, n = item.seq, item.num_new_tokens
            start = seq.num_computed_tokens
            toks = list(seq.token_ids()) + list(getattr(seq, "spec_tokens", None) or [])
            ids += toks[start: start + n]
            pos += range(start, start + n)
            q_lens.append(n)
            ctx_lens.append(start + n)
            tables.append(seq.block_table)
            last.append(len(ids) - 1)
        rows: list[int] = []
        for i in sample_rows:
            k = (num_logits or {}).get(i, 1)
            rows += range(last[i] - k + 1, last[i] + 1)
        self._check_tables(tables, ctx_lens)
        m = self.model
        self._check_ids(ids, m.cfg.vocab_size)
        # The forward always runs, also when no row is sampled: a step made only of non-final
        # prompt chunks (chunked prefill) writes its K/V here and samples nothing.
        if self._decode_step_ok(q_lens, rows):
            return self._decode(ids, ctx_lens, tables, rows)
        meta = AttentionMetadata.build(q_lens, ctx_lens, tables, self.block_size, self.device,
                                       self.attention_backend)
        hidden = m(torch.tensor(ids, dtype=torch.long, device=self.device),
                   torch.tensor(pos, dtype=torch.long, device=self.device), self.cache.layers, meta)
        if not rows:
            return torch.empty(0, m.cfg.vocab_size)
        sel = torch.tensor(rows, dtype=torch.long, device=self.device)
        return m.compute_logits(hidden.index_select(0, sel)).float().cpu()

    def _decode(self, ids, ctx_lens, tables, rows) -> torch.Tensor:
        """The fused decode step for a batch of one new token per sequence."""
        bs = self.block_size
        need = [-(-c // bs) for c in ctx_lens]
        for t, n in zip(tables, need):
            if len(t) < n:
                raise ValueError(f"block table has {len(t)} blocks, needs {n}")
        width = max(need)
        bt = np.zeros((len(tables), width), dtype=np.int64)
        for i, (t, n) in enumerate(zip(tables, need)):
            bt[i, :n] = t[:n]
        dev = self.device
        m = self.model
        B = len(ids)
        h = m.forward_decode(torch.tensor(ids, dtype=torch.long, device=dev),
                             torch.tensor(ctx_lens, dtype=torch.long, device=dev),
                             torch.from_numpy(bt).to(dev), self.cache.layers, bs)
        if not rows:
            out = torch.empty(0, m.cfg.vocab_size)
        else:
            logits = m.compute_logits(h, B if m._lm_frag(B) else None)
            out = logits.index_select(0, torch.tensor(rows, device=dev)).float().cpu()
        m.check_chain()  # after the copy's synchronization: a chain that gave up raises
        return out


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
        # The longest context a step may reach: past the block table or the RoPE table the
        # decode kernels would skip the token (its K/V unwritten, its q undefined).
        self.max_context = min(self.block_tables.shape[1] * self.block_size,
                               int(model.rope_cos.shape[0]))
        # Host copy of the longest current context (the device advances every row by one per
        # step), so that a step that would pass max_context raises before it runs.
        self._longest = int(self.context_lens.max()) if B else 0
        if self._longest > self.max_context:
            raise ValueError(f"a context of {self._longest} tokens exceeds the {self.max_context} "
                             "the block tables / RoPE table hold")
        self.logits: torch.Tensor | None = None
        self.graph: torch.cuda.CUDAGraph | None = None

    def steps_left(self) -> int:
        """Decode steps that still fit the block tables and the RoPE table."""
        return self.max_context - self._longest + 1

    def _advance(self) -> None:
        if self.steps_left() <= 0:
            raise RuntimeError(f"decode step past the longest supported context "
                               f"({self.max_context} tokens): widen the block tables")
        self._longest += 1

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
        self._advance()
        self._step()
        return self.ids

    def capture(self, keep_state: bool = True) -> None:
        """Record one step into a HIP graph. One eager step runs first, on a side stream, so
        that kernel attributes, library handles and workspaces are set up outside the graph;
        with ``keep_state`` the ids, context lengths and caches are restored after it, else
        that step counts as a decoded token."""
        saved = self.snapshot() if keep_state else None
        self._advance()
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
        self._longest = int(ctx.max()) if ctx.numel() else 0
        for (k, v), (kd, ks, vd, vs) in zip(self.cache.layers, layers, strict=True):
            k.data.copy_(kd)
            k.scale.copy_(ks)
            v.data.copy_(vd)
            v.scale.copy_(vs)

    def replay(self) -> torch.Tensor:
        """One graph replay = one decode step; returns the ids buffer."""
        if self.graph is None:
            raise RuntimeError("capture() first")
        self._advance()
        self.graph.replay()
        return self.ids

    def check(self) -> None:
        """Raises when a decode-chain launch of the steps since the last check gave up on a
        hand-off wait (the tokens those steps produced are invalid). ``step`` and ``replay``
        never synchronize; a caller that reads the ids on the host calls this alongside.
        Synchronizes."""
        if getattr(self.model, "_chain_ws", None) is not None:
            self.model._chain_pending = True  # graph replays launch the chain without the flag
        self.model.check_chain()
