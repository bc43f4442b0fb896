"""Paged attention over a block-structured KV cache, with the int8 cache on MI355X.

Drop-in for the reference's ``llmserve.attention`` (src/llmserve/attention.py). The engine
runs one forward pass over a ragged batch whose new tokens are concatenated into ``[T]``; the
KV of every sequence lives in fixed-size blocks addressed through a block table, and a cache
slot is ``block_id * block_size + offset``.

On a ROCm device with an int8 cache (``QuantizedKV``) and the native backend:
  * the new K/V rows are quantized and scattered by one HIP kernel per tensor (key smoothing
    ``k / s`` fused into the key's kernel),
  * decode rows run the split-context int8 paged-decode HIP kernel, with the smoothing
    multiply ``q * s`` fused into its q load.
Prefill rows (several new tokens) gather the dequantized context and call SDPA, as the
reference does (attention.py:249-257). The native backend is named "hip"; "cpp" (the
reference's name) is accepted as an alias.
"""

from __future__ import annotations

import functools
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

NATIVE_BACKENDS = ("hip", "cpp")


@dataclass
class PrefillSeq:
    q_start: int  # offset of this sequence's first new token in the flat batch
    q_len: int  # number of new tokens
    ctx_len: int  # total tokens attended to = cached + new
    slots: torch.Tensor  # [ctx_len] cache slots of the whole context, in order


@dataclass
class AttentionMetadata:
    """Per-step attention metadata, shared by all layers (reference attention.py:33-124)."""

    slot_mapping: torch.Tensor  # [T]
    prefills: list[PrefillSeq] = field(default_factory=list)
    decode_token_idx: torch.Tensor | None = None  # [Bd] index into the flat batch
    decode_block_tables: torch.Tensor | None = None  # [Bd, max_blocks] (native kernel)
    decode_ctx_lens: torch.Tensor | None = None  # [Bd]
    decode_slots: torch.Tensor | None = None  # [Bd, max_ctx] (torch path)
    decode_mask: torch.Tensor | None = None  # [Bd, 1, 1, max_ctx] True = attend (torch path)
    block_size: int = 16
    backend: str = "torch"  # "torch" (gather + SDPA) or "hip"/"cpp" (native paged kernel)
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
        """``q_lens[i]`` new tokens of sequence ``i`` sit at the end of its ``ctx_lens[i]``-token
        context; ``block_tables[i]`` lists the physical blocks holding that context."""
        slot_parts: list[torch.Tensor] = []
        prefills: list[PrefillSeq] = []
        dec_idx: list[int] = []
        dec_slots: list[torch.Tensor] = []
        dec_tables: list[list[int]] = []
        dec_ctx: list[int] = []
        q_start = 0
        for q_len, ctx_len, table in zip(q_lens, ctx_lens, block_tables, strict=True):
            n_blocks = (ctx_len + block_size - 1) // block_size
            if len(table) < n_blocks:
                raise ValueError(f"block table has {len(table)} blocks, needs {n_blocks}")
            blocks = torch.tensor(table[:n_blocks], dtype=torch.long)
            slots = (
                blocks[:, None] * block_size + torch.arange(block_size, dtype=torch.long)
            ).flatten()[:ctx_len]
            slot_parts.append(slots[ctx_len - q_len :])
            if q_len == 1:
                dec_idx.append(q_start)
                dec_slots.append(slots)
                dec_tables.append(table[:n_blocks])
                dec_ctx.append(ctx_len)
            else:
                prefills.append(PrefillSeq(q_start, q_len, ctx_len, slots.to(device)))
            q_start += q_len

        native = backend in NATIVE_BACKENDS
        meta = AttentionMetadata(
            slot_mapping=torch.cat(slot_parts).to(device)
            if slot_parts
            else torch.empty(0, dtype=torch.long, device=device),
            prefills=prefills,
            block_size=block_size,
            backend="hip" if native else backend,
        )
        if dec_idx and native:
            mb = max(len(t) for t in dec_tables)
            bt = torch.zeros(len(dec_tables), mb, dtype=torch.long)
            for i, t in enumerate(dec_tables):
                bt[i, : len(t)] = torch.tensor(t, dtype=torch.long)
            meta.decode_token_idx = torch.tensor(dec_idx, dtype=torch.long, device=device)
            meta.decode_block_tables = bt.to(device)
            meta.decode_ctx_lens = torch.tensor(dec_ctx, dtype=torch.long, device=device)
        elif dec_idx:
            max_ctx = max(s.numel() for s in dec_slots)
            table = torch.zeros(len(dec_slots), max_ctx, dtype=torch.long)
            mask = torch.zeros(len(dec_slots), max_ctx, dtype=torch.bool)
            for i, s in enumerate(dec_slots):
                table[i, : s.numel()] = s
                mask[i, : s.numel()] = True
            meta.decode_token_idx = torch.tensor(dec_idx, dtype=torch.long, device=device)
            meta.decode_slots = table.to(device)
            meta.decode_mask = mask[:, None, None, :].to(device)
        return meta

    def prefill_mask(self, i: int) -> torch.Tensor | None:
        """Causal mask for prefill sequence ``i`` when part of its context is already cached."""
        if i not in self._prefill_masks:
            p = self.prefills[i]
            if p.q_len == p.ctx_len:
                self._prefill_masks[i] = None  # plain causal; use is_causal fast path
            else:
                q_pos = torch.arange(p.ctx_len - p.q_len, p.ctx_len, device=p.slots.device)
                k_pos = torch.arange(p.ctx_len, device=p.slots.device)
                self._prefill_masks[i] = k_pos[None, :] <= q_pos[:, None]
        return self._prefill_masks[i]


class QuantizedKV:
    """One layer's K (or V) cache as int8 with one fp32 scale per (token slot, kv head)
    (reference attention.py:127-173).

    Symmetric absmax quantization ``x ~= data * scale``, ``scale = max(max|x|, 1e-8) / 127``
    over the head dimension, computed by the ``llmserve_kv_quantize_write`` HIP kernel with
    the reference's CPU arithmetic (clamp, then divide; round half to even).
    """

    # Validate slot indices on the host before a write (one device sync per write). The
    # kernel itself skips out-of-range slots; torch.index_copy_ would raise for them.
    check_slots = False

    def __init__(self, num_slots: int, kv_heads: int, head_dim: int, device="cpu") -> None:
        self.data = torch.zeros(num_slots, kv_heads, head_dim, dtype=torch.int8, device=device)
        self.scale = torch.zeros(num_slots, kv_heads, dtype=torch.float32, device=device)
        self.smooth: torch.Tensor | None = None  # [kv_heads, head_dim]
        self._q_mult: torch.Tensor | None = None  # [q_heads, head_dim]

    def set_smoothing(self, s: torch.Tensor | None, num_q_heads: int) -> None:
        """SmoothQuant-style key smoothing: store ``k / s`` and attend with ``q * s``
        (reference attention.py:142-151)."""
        if s is not None:
            s = s.to(device=self.data.device, dtype=torch.float32).contiguous()
        self.smooth = s
        g = num_q_heads // s.shape[0] if s is not None else 1
        self._q_mult = s.repeat_interleave(g, 0).contiguous() if s is not None else None

    @staticmethod
    def quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(int8 data, fp32 scale) of ``x`` [..., D], scale over the last dimension."""
        from llmserve.kernels import load_quant

        x = x.float().contiguous()
        lead, D = x.shape[:-1], x.shape[-1]
        x3 = x.reshape(-1, 1, D)
        n = x3.shape[0]
        data = torch.empty(n, 1, D, dtype=torch.int8, device=x.device)
        scale = torch.empty(n, 1, dtype=torch.float32, device=x.device)
        slots = torch.arange(n, dtype=torch.long, device=x.device)
        load_quant().kv_quantize_write(x3, slots, data, scale, None)
        return data.reshape(*lead, D), scale.reshape(lead)

    def write(self, slots: torch.Tensor, x: torch.Tensor, smooth: torch.Tensor | None = None) -> None:
        """Quantize ``x`` [T, Hk, D] into ``slots`` [T]; with ``smooth`` the rows written are
        ``x / smooth`` (the division fused into the kernel)."""
        from llmserve.kernels import load_quant

        slots = slots.to(device=self.data.device, dtype=torch.long).contiguous()
        if self.check_slots and slots.numel():
            lo, hi = int(slots.min()), int(slots.max())
            if lo < 0 or hi >= self.data.shape[0]:
                raise IndexError(f"slot index out of range [0, {self.data.shape[0]})")
        load_quant().kv_quantize_write(x.float().contiguous(), slots, self.data, self.scale, smooth)

    def rows(self, idx: torch.Tensor) -> torch.Tensor:
        """Dequantized rows (float32) for slot indices of any shape."""
        return self.data[idx].float() * self.scale[idx].unsqueeze(-1)

    def copy_rows(self, dst: torch.Tensor, src: torch.Tensor) -> None:
        self.data[dst] = self.data[src]
        self.scale[dst] = self.scale[src]

    def nbytes(self) -> int:
        return self.data.numel() + self.scale.numel() * 4


_K_STATS: list | None = None


def smoothing_from_stats(stats: list[torch.Tensor], alpha: float = 1.0) -> list[torch.Tensor]:
    """Per-layer factors ``s = clamp(max|K|, 1e-5) ** alpha`` normalised to mean 1 per head
    (reference attention.py:196-200)."""
    out = []
    for m in stats:  # [Hk, D]
        s = m.float().clamp_min(1e-5).pow(alpha)
        out.append(s / s.mean(-1, keepdim=True))
    return out


@torch.inference_mode()
def calibrate_k_smoothing(model, ids: list[int], alpha: float = 1.0) -> list[torch.Tensor]:
    """Key smoothing factors from one fp32 prefill of ``ids`` (reference attention.py:179-200).
    ``model`` follows the reference's calling convention ``model(ids, pos, kv_caches, meta)``
    and carries ``cfg``."""
    global _K_STATS
    from llmserve.kv_cache import KVCache

    bs = 16
    nb = -(-len(ids) // bs)
    p0 = next(model.parameters())
    cache = KVCache(model.cfg, nb, bs, p0.dtype, device=p0.device)
    meta = AttentionMetadata.build([len(ids)], [len(ids)], [list(range(nb))], bs, device=p0.device)
    _K_STATS = []
    try:
        model(torch.tensor(ids, device=p0.device), torch.arange(len(ids), device=p0.device),
              cache.layers, meta)
        stats = _K_STATS
    finally:
        _K_STATS = None
    return smoothing_from_stats(stats, alpha)


# A fixed, generic calibration text (the reference's attention.py:204-214).
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


def _rows(cache, idx: torch.Tensor) -> torch.Tensor:
    return cache.rows(idx) if isinstance(cache, QuantizedKV) else cache[idx]


def write_kv(k_cache, v_cache, k: torch.Tensor, v: torch.Tensor, slots: torch.Tensor) -> None:
    """Scatter new K/V ([T, Hk, D]) into flat cache tensors ([num_slots, Hk, D])."""
    if isinstance(k_cache, QuantizedKV):
        k_cache.write(slots, k)
        v_cache.write(slots, v)
        return
    k_cache.index_copy_(0, slots, k)
    v_cache.index_copy_(0, slots, v)


def paged_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    k_cache,
    v_cache,
    meta: AttentionMetadata,
    scale: float,
) -> torch.Tensor:
    """Write this step's K/V into the cache, then attend. q: [T, Hq, D] -> out: [T, Hq, D]
    (reference attention.py:231-307)."""
    if _K_STATS is not None:  # calibration pass (calibrate_k_smoothing)
        _K_STATS.append(k.detach().abs().amax(0))
    quantized = isinstance(k_cache, QuantizedKV)
    smooth = k_cache.smooth if quantized else None
    if quantized:
        k_cache.write(meta.slot_mapping, k, smooth)  # k / smooth fused in the kernel
        v_cache.write(meta.slot_mapping, v)
    else:
        write_kv(k_cache, v_cache, k, v, meta.slot_mapping)
    # q * s for the torch paths; the native decode kernel applies the same product itself
    q_s = q * k_cache._q_mult if smooth is not None else q
    out = q.new_empty(q.shape)

    for i, p in enumerate(meta.prefills):
        qi = q_s[p.q_start : p.q_start + p.q_len].transpose(0, 1).unsqueeze(0)  # [1, Hq, q, D]
        ki = _rows(k_cache, p.slots).transpose(0, 1).unsqueeze(0)  # [1, Hk, ctx, D]
        vi = _rows(v_cache, p.slots).transpose(0, 1).unsqueeze(0)
        mask = meta.prefill_mask(i)
        oi = F.scaled_dot_product_attention(
            qi, ki, vi, attn_mask=mask, is_causal=mask is None, scale=scale, enable_gqa=True
        )
        out[p.q_start : p.q_start + p.q_len] = oi.squeeze(0).transpose(0, 1)

    if meta.decode_block_tables is not None:
        if not quantized:
            raise NotImplementedError(
                "the native decode kernel serves the int8 KV cache; use backend='torch' "
                "for an fp32 cache"
            )
        from llmserve.kernels import load_paged_attention

        od = load_paged_attention().paged_attention_decode_int8(
            q[meta.decode_token_idx].contiguous(),
            k_cache.data,
            v_cache.data,
            k_cache.scale,
            v_cache.scale,
            meta.decode_block_tables,
            meta.decode_ctx_lens,
            meta.block_size,
            scale,
            0,
            k_cache._q_mult,
        )
        if not meta.prefills:
            return od
        out[meta.decode_token_idx] = od
    elif meta.decode_token_idx is not None:
        qd = q_s[meta.decode_token_idx].unsqueeze(2)  # [B, Hq, 1, D]
        kd = _rows(k_cache, meta.decode_slots).transpose(1, 2)  # [B, Hk, ctx, D]
        vd = _rows(v_cache, meta.decode_slots).transpose(1, 2)
        od = F.scaled_dot_product_attention(
            qd, kd, vd, attn_mask=meta.decode_mask, scale=scale, enable_gqa=True
        )
        out[meta.decode_token_idx] = od.squeeze(2)
    return out


@functools.cache
def resolve_backend(name: str, device: str = "cpu") -> str:
    """``auto`` -> ``hip`` on a ROCm device when the native library loads, else ``torch``
    (reference attention.py:310-323, where the native kernel was CPU-only)."""
    if name == "torch":
        return "torch"
    if name not in ("auto",) + NATIVE_BACKENDS:
        raise ValueError(f"unknown attention backend {name!r}")
    from llmserve.kernels import NativeLibraryMissing, load_paged_attention

    on_gpu = str(device).startswith("cuda")
    if on_gpu:
        try:
            load_paged_attention()
            return "hip"
        except NativeLibraryMissing:
            if name != "auto":
                raise
    if name != "auto":
        raise RuntimeError("native paged attention kernel needs a ROCm device")
    return "torch"
