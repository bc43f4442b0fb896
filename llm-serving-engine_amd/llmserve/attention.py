"""Paged attention over a block-structured KV cache, with the native path on MI355X.

Drop-in for the reference's ``llmserve.attention`` (src/llmserve/attention.py): the same
classes, fields and functions. A step runs one forward pass over a ragged batch whose new tokens
are laid end to end in a flat ``[T]`` stream; every sequence keeps its K/V in fixed-size blocks
listed by its block table, and cache slot = ``block_id * block_size + offset``.

Two backends, chosen by ``AttentionMetadata.backend``:

* ``"hip"`` (alias ``"cpp"``, the reference's name for its native kernel), on a ROCm device:
  ``AttentionMetadata.build`` packs the block tables once on the host and a HIP kernel derives
  the slot of every new token and its *query row*: the block-table row it attends over and how
  many tokens it sees (its position + 1, the causal mask). ``paged_attention`` then writes the
  new K/V (int8 caches: one quantize-and-scatter kernel per tensor, key smoothing ``k / s``
  fused) and runs ONE split-context paged attention launch over all T rows, decode and prefill
  alike, int8 or fp32 cache, with the smoothing product ``q * s`` fused into its q load.
* ``"torch"``: slots and per-sequence tables are computed with vectorised numpy on the host;
  attention gathers the (dequantized) context rows and calls SDPA, the reference's algorithm
  (attention.py:249-257, :299-306).
"""

from __future__ import annotations

import contextlib
import functools
import itertools
from dataclasses import dataclass, field

import numpy as np
import torch
import torch.nn.functional as F

NATIVE_BACKENDS = ("hip", "cpp")


@dataclass
class PrefillSeq:
    """A sequence with several new tokens in this step (a prompt chunk)."""

    q_start: int  # index of its first new token in the flat batch
    q_len: int  # how many new tokens it has
    ctx_len: int  # tokens it attends to: the cached ones plus the new ones
    slots: torch.Tensor  # [ctx_len] the cache slot of each context position, in order


@dataclass
class AttentionMetadata:
    """What every layer of one step needs to know about the batch (reference
    attention.py:33-124). Built once per step and shared by all layers."""

    slot_mapping: torch.Tensor  # [T] cache slot each new token's K/V is written to
    prefills: list[PrefillSeq] = field(default_factory=list)
    decode_token_idx: torch.Tensor | None = None  # [Bd] flat index of each decode token
    decode_block_tables: torch.Tensor | None = None  # [Bd, max_blocks] zero-padded (native)
    decode_ctx_lens: torch.Tensor | None = None  # [Bd]
    decode_slots: torch.Tensor | None = None  # [Bd, max_ctx] slot table (torch backend)
    decode_mask: torch.Tensor | None = None  # [Bd, 1, 1, max_ctx] True where attended (torch)
    block_size: int = 16
    backend: str = "torch"  # "torch" or "hip" ("cpp" accepted as an alias)
    # Native backend: every token is one query row of the paged attention kernel.
    block_tables: torch.Tensor | None = None  # [S, max_blocks] the batch's tables, zero-padded
    row_table: torch.Tensor | None = None  # [T] the table row token t attends over
    row_context: torch.Tensor | None = None  # [T] how many context tokens token t sees
    _prefill_masks: dict[int, torch.Tensor | None] = field(default_factory=dict)

    @staticmethod
    def build(
        q_lens: list[int],
        ctx_lens: list[int],
        block_tables: list[list[int]],
        block_size: int,
        device: torch.device | str = "cpu",
        backend: str = "torch",
    ) -> AttentionMetadata:
        """``q_lens[i]`` new tokens of sequence ``i`` are the last ones of its ``ctx_lens[i]``
        tokens; ``block_tables[i]`` lists the physical blocks of that context in order."""
        plan = _BatchPlan(q_lens, ctx_lens, block_tables, block_size)
        native = backend in NATIVE_BACKENDS
        meta = AttentionMetadata(slot_mapping=torch.empty(0, dtype=torch.long, device=device),
                                 block_size=block_size, backend="hip" if native else backend)
        if native and _native_ops(device) is not None:
            plan.fill_native(meta, device)
        else:
            plan.fill_host(meta, device, native)
        return meta

    def prefill_mask(self, i: int) -> torch.Tensor | None:
        """Boolean [q_len, ctx_len] causal mask of prefill sequence ``i`` (None when nothing of
        it was cached, so that SDPA's ``is_causal`` applies); cached per sequence."""
        if i not in self._prefill_masks:
            p = self.prefills[i]
            mask = None
            if p.q_len != p.ctx_len:
                dev = p.slots.device
                first = p.ctx_len - p.q_len  # position of the first new token
                mask = (torch.arange(p.ctx_len, device=dev)[None, :]
                        <= torch.arange(first, p.ctx_len, device=dev)[:, None])
            self._prefill_masks[i] = mask
        return self._prefill_masks[i]


class _BatchPlan:
    """The batch of one step as numpy arrays: sizes, token offsets and the packed tables."""

    def __init__(self, q_lens, ctx_lens, block_tables, block_size: int) -> None:
        if not len(q_lens) == len(ctx_lens) == len(block_tables):
            raise ValueError("q_lens, ctx_lens and block_tables must have one entry per sequence")
        self.bs = int(block_size)
        self.q = np.asarray(q_lens, dtype=np.int64).reshape(-1)
        self.ctx = np.asarray(ctx_lens, dtype=np.int64).reshape(-1)
        self.S = self.q.size
        need = (self.ctx + self.bs - 1) // self.bs
        have = np.fromiter((len(t) for t in block_tables), dtype=np.int64, count=self.S)
        short = np.flatnonzero(have < need)
        if short.size:
            i = short[0]
            raise ValueError(f"block table has {have[i]} blocks, needs {need[i]}")
        self.width = max(1, int(need.max())) if self.S else 1
        self.tables = np.zeros((self.S, self.width), dtype=np.int64)
        used = np.arange(self.width)[None, :] < need[:, None]
        self.tables[used] = np.fromiter(
            itertools.chain.from_iterable(t[:n] for t, n in zip(block_tables, need.tolist())),
            dtype=np.int64, count=int(need.sum()))
        self.q_start = np.cumsum(self.q) - self.q
        self.T = int(self.q.sum())
        self.dec = np.flatnonzero(self.q == 1)  # decode sequences
        self.pre = np.flatnonzero(self.q != 1)  # prefill sequences (several new tokens)

    def slots_of(self, seq: np.ndarray, pos: np.ndarray) -> np.ndarray:
        """Cache slots of positions ``pos`` of sequences ``seq`` (broadcasting)."""
        return self.tables[seq, pos // self.bs] * self.bs + pos % self.bs

    def token_positions(self) -> tuple[np.ndarray, np.ndarray]:
        """(sequence, position) of every new token of the flat batch."""
        seq = np.repeat(np.arange(self.S), self.q)
        pos = self.ctx[seq] - self.q[seq] + (np.arange(self.T) - self.q_start[seq])
        return seq, pos

    def prefill_seqs(self, device, tables_dev: torch.Tensor | None) -> list[PrefillSeq]:
        out = []
        for s in self.pre.tolist():
            c = int(self.ctx[s])
            if tables_dev is not None:  # on the device, from the uploaded tables
                pos = torch.arange(c, device=tables_dev.device)
                slots = tables_dev[s, pos // self.bs] * self.bs + pos % self.bs
            else:
                slots = torch.from_numpy(self.slots_of(np.int64(s), np.arange(c))).to(device)
            out.append(PrefillSeq(int(self.q_start[s]), int(self.q[s]), c, slots))
        return out

    def fill_host(self, meta: AttentionMetadata, device, native: bool = False) -> None:
        """Everything computed with numpy, then copied to ``device``: the decode rows as
        zero-padded block tables for a native backend (the reference's fields for its kernel),
        as a slot table and mask for the torch backend."""
        seq, pos = self.token_positions()
        meta.slot_mapping = torch.from_numpy(self.slots_of(seq, pos)).to(device)
        meta.prefills = self.prefill_seqs(device, None)
        if self.dec.size and native:
            ctx = self.ctx[self.dec]
            width = int(((ctx + self.bs - 1) // self.bs).max())
            meta.decode_token_idx = torch.from_numpy(self.q_start[self.dec]).to(device)
            meta.decode_block_tables = torch.from_numpy(self.tables[self.dec, :width].copy()).to(device)
            meta.decode_ctx_lens = torch.from_numpy(ctx).to(device)
        elif self.dec.size:
            ctx = self.ctx[self.dec]
            span = np.arange(int(ctx.max()))
            inside = span[None, :] < ctx[:, None]
            slots = np.where(inside, self.slots_of(self.dec[:, None], np.minimum(span, ctx[:, None] - 1)), 0)
            meta.decode_token_idx = torch.from_numpy(self.q_start[self.dec]).to(device)
            meta.decode_slots = torch.from_numpy(slots).to(device)
            meta.decode_mask = torch.from_numpy(inside)[:, None, None, :].to(device)

    def fill_native(self, meta: AttentionMetadata, device) -> None:
        """Native backend: one upload of the packed batch, then the metadata kernel."""
        info = np.concatenate([self.q, self.ctx, self.q_start, self.tables.reshape(-1)])
        dev_info = torch.from_numpy(info).to(device)
        seq_info = dev_info[: 3 * self.S].view(3, self.S)
        tables = dev_info[3 * self.S:].view(self.S, self.width)
        meta.block_tables = tables
        if self.T:
            meta.slot_mapping, meta.row_table, meta.row_context = _native_ops(device).attention_metadata(
                seq_info, tables, self.bs, self.T)
        meta.prefills = self.prefill_seqs(device, tables)
        if self.dec.size:
            dec = torch.from_numpy(self.dec).to(device)
            meta.decode_token_idx = seq_info[2].index_select(0, dec)
            meta.decode_block_tables = tables.index_select(0, dec)
            meta.decode_ctx_lens = seq_info[1].index_select(0, dec)


@functools.cache
def _ops_namespace():
    from .kernels import load_paged_attention

    return load_paged_attention()


def _native_ops(device):
    """The native attention ops when they can run on ``device`` (a ROCm device with the
    library built), else None."""
    if torch.device(device).type != "cuda":
        return None
    return _ops_namespace()


# ---- int8 cache ------------------------------------------------------------------------------


def _kv_int8_torch(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric int8 with torch ops: scale = max(max|x|, 1e-8) / 127 (the clamp comes
    before the division, attention.py:156), q = clamp(round_half_even(x / scale), +-127)."""
    scale = torch.clamp(x.abs().amax(dim=-1), min=1e-8) / 127.0
    q = torch.clamp(torch.round(x / scale.unsqueeze(-1)), -127, 127).to(torch.int8)
    return q, scale


class QuantizedKV:
    """One layer's K (or V) cache as int8 plus one fp32 scale per (slot, kv head) (reference
    attention.py:127-173): ``row ~= data * scale``, ``scale = max(max|row|, 1e-8) / 127`` over
    the head dimension. On a ROCm device the quantize-and-scatter is the
    ``llmserve_kv_quantize_write`` HIP kernel (bit-identical to the torch CPU ops); elsewhere,
    or without the native library, torch ops compute it.
    """

    # Check slot indices on the host before a native write (one device sync per write); the
    # kernel skips slots outside the cache, where torch.index_copy_ would raise.
    check_slots = False

    def __init__(self, num_slots: int, kv_heads: int, head_dim: int, device="cpu") -> None:
        shape = (num_slots, kv_heads)
        self.data = torch.zeros(shape + (head_dim,), dtype=torch.int8, device=device)
        self.scale = torch.zeros(shape, dtype=torch.float32, device=device)
        self.smooth: torch.Tensor | None = None  # [kv_heads, head_dim] (K cache only)
        self._q_mult: torch.Tensor | None = None  # [q_heads, head_dim]: smooth per query head

    def set_smoothing(self, s: torch.Tensor | None, num_q_heads: int) -> None:
        """Key smoothing (SmoothQuant-style, reference attention.py:142-151): the cache stores
        ``k / s`` and attention uses ``q * s``, which leaves q . k unchanged in exact arithmetic
        while the few large key channels stop setting every row's int8 scale."""
        if s is None:
            self.smooth = self._q_mult = None
            return
        s = s.to(device=self.data.device, dtype=torch.float32).contiguous()
        group = num_q_heads // s.shape[0]
        self.smooth = s
        self._q_mult = torch.repeat_interleave(s, group, dim=0).contiguous()

    @staticmethod
    def quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(int8 data, fp32 scale) of ``x`` [..., D], one scale per row of D values."""
        x = x.float().contiguous()
        ops = _quant_ops(x)
        if ops is None:
            return _kv_int8_torch(x)
        rows = x.reshape(-1, 1, x.shape[-1])
        n = rows.shape[0]
        data = torch.empty(rows.shape, dtype=torch.int8, device=x.device)
        scale = torch.empty(n, 1, dtype=torch.float32, device=x.device)
        ops.kv_quantize_write(rows, torch.arange(n, device=x.device), data, scale, None)
        return data.view(x.shape), scale.view(x.shape[:-1])

    def write(self, slots: torch.Tensor, x: torch.Tensor,
              smooth: torch.Tensor | None = None) -> None:
        """Quantize ``x`` [T, Hk, D] (divided by ``smooth`` first when given) into ``slots``."""
        x = x.float().contiguous()
        slots = slots.to(device=self.data.device, dtype=torch.long).contiguous()
        ops = _quant_ops(x)
        if ops is None:
            q, s = _kv_int8_torch(x / smooth if smooth is not None else x)
            self.data.index_copy_(0, slots, q)
            self.scale.index_copy_(0, slots, s)
            return
        if self.check_slots and slots.numel():
            bad = (slots < 0) | (slots >= self.data.shape[0])
            if bool(bad.any()):
                raise IndexError(f"slot index out of range [0, {self.data.shape[0]})")
        ops.kv_quantize_write(x, slots, self.data, self.scale, smooth)

    def rows(self, idx: torch.Tensor) -> torch.Tensor:
        """Dequantized float32 rows for slot indices of any shape."""
        return torch.mul(self.data[idx].to(torch.float32), self.scale[idx][..., None])

    def copy_rows(self, dst: torch.Tensor, src: torch.Tensor) -> None:
        """Copy whole slot rows (data and scales) from ``src`` to ``dst`` (block copies)."""
        for t in (self.data, self.scale):
            t.index_copy_(0, dst.to(t.device), t.index_select(0, src.to(t.device)))

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.data, self.scale))


def _quant_ops(x: torch.Tensor):
    if not x.is_cuda:
        return None
    from .kernels import load_quant

    return load_quant()


# ---- key smoothing calibration -----------------------------------------------------------------

_K_STATS: list | None = None


def smoothing_from_stats(stats: list[torch.Tensor], alpha: float = 1.0) -> list[torch.Tensor]:
    """Per-layer smoothing factors from per-layer max|K| [Hk, D] (reference attention.py:
    196-200): ``s = max(max|K|, 1e-5) ** alpha``, divided by its mean over D per head."""
    factors = []
    for amax in stats:
        s = torch.pow(torch.clamp(amax.float(), min=1e-5), alpha)
        factors.append(s / torch.mean(s, dim=-1, keepdim=True))
    return factors


@contextlib.contextmanager
def _recording_key_stats():
    """While active, ``paged_attention`` appends each layer's max|K| over the batch."""
    global _K_STATS
    _K_STATS = stats = []
    try:
        yield stats
    finally:
        _K_STATS = None


def _model_placement(model) -> tuple[torch.device, torch.dtype]:
    for t in itertools.chain(model.parameters(), model.buffers()):
        if t is not None and t.is_floating_point():
            return t.device, t.dtype
    return torch.device("cpu"), torch.float32


@torch.inference_mode()
def calibrate_k_smoothing(model, ids: list[int], alpha: float = 1.0) -> list[torch.Tensor]:
    """Key smoothing factors from one fp32 prefill of ``ids`` (reference attention.py:179-200).
    ``model`` has the reference's calling convention ``model(ids, positions, kv_caches, meta)``
    and a ``cfg``; the prefill runs over a throw-away cache in the model's dtype on its device
    (``QuantCausalLM`` of this package qualifies)."""
    from .kv_cache import KVCache

    dev, dtype = _model_placement(model)
    bs = 16
    n_blocks = max(1, -(-len(ids) // bs))
    cache = KVCache(model.cfg, n_blocks, bs, dtype, device=dev)
    backend = resolve_backend("auto", str(dev))
    meta = AttentionMetadata.build([len(ids)], [len(ids)], [list(range(n_blocks))], bs, dev, backend)
    with _recording_key_stats() as stats:
        model(torch.as_tensor(ids, dtype=torch.long, device=dev),
              torch.arange(len(ids), device=dev), cache.layers, meta)
    return smoothing_from_stats(stats, alpha)


# A fixed, generic calibration text (the reference's attention.py:204-214; data the
# calibration must reproduce).
CALIBRATION_TEXT = (
    "The history of computing is a story of people trying to make machines do useful work. "
    "Early mechanical calculators added and multiplied numbers with gears; later, electronic "
    "computers stored programs in memory and ran them at speeds no clerk could match. Today a "
    "phone holds more processing power than the rooms of equipment that guided the first "
    "spacecraft. Software grew alongside the hardware: operating systems, compilers, databases "
    "and networks turned raw circuits into tools for writing, science, trade and art. "
    "Questions people ask an assistant range from recipes and travel plans to code reviews, "
    "math homework and medical worries, so a language model must handle plain conversation, "
    "lists, numbers like 3.14 or 2024, and snippets such as def add(a, b): return a + b."
)


# ---- attention -----------------------------------------------------------------------------------


def write_kv(k_cache, v_cache, k: torch.Tensor, v: torch.Tensor, slots: torch.Tensor) -> None:
    """Store this step's K/V rows ([T, Hk, D]) at ``slots`` of flat fp32 or int8 caches."""
    for cache, rows in ((k_cache, k), (v_cache, v)):
        if isinstance(cache, QuantizedKV):
            cache.write(slots, rows)
        else:
            cache.index_copy_(0, slots, rows.to(cache.dtype))


def _context(cache, idx: torch.Tensor) -> torch.Tensor:
    """Float rows of the cache at slot indices ``idx`` ([..., Hk, D])."""
    return cache.rows(idx) if isinstance(cache, QuantizedKV) else cache[idx]


def _sdpa_heads_first(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask, scale: float,
                      causal: bool = False) -> torch.Tensor:
    """SDPA over rows laid out [(B,) L, H, D] (heads second to last), GQA allowed."""
    single = q.dim() == 3
    if single:
        q, k, v = q[None], k[None], v[None]
    o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                       attn_mask=mask, is_causal=causal, scale=scale,
                                       enable_gqa=True).transpose(1, 2)
    return o[0] if single else o


def _attend_torch(q: torch.Tensor, k_cache, v_cache, meta: AttentionMetadata, scale: float,
                  out: torch.Tensor) -> None:
    """The gather + SDPA algorithm of the reference (attention.py:249-257, :299-306)."""
    for i, p in enumerate(meta.prefills):
        rows = slice(p.q_start, p.q_start + p.q_len)
        mask = meta.prefill_mask(i)
        out[rows] = _sdpa_heads_first(q[rows], _context(k_cache, p.slots),
                                      _context(v_cache, p.slots), mask, scale, mask is None)
    if meta.decode_token_idx is None:
        return
    idx = meta.decode_token_idx
    if meta.decode_slots is None:  # a native plan attended with torch: derive the slot table
        span = torch.arange(int(meta.decode_ctx_lens.max()), device=idx.device)
        inside = span[None, :] < meta.decode_ctx_lens[:, None]
        pos = torch.minimum(span[None, :], meta.decode_ctx_lens[:, None] - 1)
        slots = torch.where(inside, torch.gather(meta.decode_block_tables, 1,
                                                 pos // meta.block_size) * meta.block_size
                            + pos % meta.block_size, 0)
        mask = inside[:, None, None, :]
    else:
        slots, mask = meta.decode_slots, meta.decode_mask
    od = _sdpa_heads_first(q[idx].unsqueeze(1), _context(k_cache, slots),
                           _context(v_cache, slots), mask, scale)
    out[idx] = od.squeeze(1)


def paged_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    k_cache,
    v_cache,
    meta: AttentionMetadata,
    scale: float,
) -> torch.Tensor:
    """Store this step's K/V in the cache, then attend: q [T, Hq, D] -> [T, Hq, D] (reference
    attention.py:231-307)."""
    if _K_STATS is not None:  # calibrate_k_smoothing is recording
        _K_STATS.append(torch.amax(k.detach().abs(), dim=0))
    quantized = isinstance(k_cache, QuantizedKV)
    smooth = k_cache.smooth if quantized else None
    ops = None
    if meta.row_table is not None and (quantized or k_cache.dtype == torch.float32):
        ops = _native_ops(q.device)
    if quantized:
        k_cache.write(meta.slot_mapping, k, smooth)  # the kernel divides by smooth
        v_cache.write(meta.slot_mapping, v)
    else:
        write_kv(k_cache, v_cache, k, v, meta.slot_mapping)
    if ops is not None:  # every token is a query row of one native launch
        q_mult = k_cache._q_mult if smooth is not None else None
        if quantized:
            return ops.paged_attention_rows(q.float().contiguous(), k_cache.data, v_cache.data,
                                            k_cache.scale, v_cache.scale, meta.block_tables,
                                            meta.row_table, meta.row_context, meta.block_size,
                                            scale, q_mult)
        return ops.paged_attention_rows(q.float().contiguous(), k_cache, v_cache, None, None,
                                        meta.block_tables, meta.row_table, meta.row_context,
                                        meta.block_size, scale, None)
    q_att = q * k_cache._q_mult if smooth is not None else q
    out = torch.empty_like(q)
    _attend_torch(q_att, k_cache, v_cache, meta, scale, out)
    return out


@functools.cache
def resolve_backend(name: str, device: str = "cpu") -> str:
    """``auto`` -> ``hip`` on a ROCm device when the native library loads, else ``torch``
    (reference attention.py:310-323, whose native kernel ran on the CPU)."""
    if name == "torch":
        return "torch"
    if name != "auto" and name not in NATIVE_BACKENDS:
        raise ValueError(f"unknown attention backend {name!r}")
    if _native_ops(device) is not None:
        return "hip"
    if name != "auto":
        raise RuntimeError("native paged attention kernel is not available (it needs a ROCm "
                           "device and the built llmserve library)")
    return "torch"
