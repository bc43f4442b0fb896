"""Quantized decoder-only model (Llama / Qwen3 layout) for the decode step on MI355X.

Mirrors the reference's ``CausalLM`` (src/llmserve/models/transformer.py:106-193) with the
linears swapped for ``Int4Linear`` (``quantize_model(method="int4-awq")``, quant.py:173-205)
and the fused forward of ``_forward_fused`` (transformer.py:144-190), restricted to a batch of
decode tokens over an int8 paged KV cache. Every op runs as a HIP kernel of this package:

  embed_rmsnorm                      embedding row + layer 0's input norm (:151-155)
  per layer:
    qkv_proj                         Int4Linear (GEMV for <= 16 rows, matrix cores above)
    decode_qkv_kv                    q/k RMSNorm + RoPE at position ctx - 1 + k / smooth +
                                     int8 quantize-write of K and V (:157-171, attention.py:241-246)
    paged_attention_decode_int8      split-context int8 decode, q * q_mult fused (attention.py:263-273)
    o_proj, add_rmsnorm_             (:183-184)
    gate_up_proj, silu_mul, down_proj, add_rmsnorm_ with the next norm   (:185-189)
  lm_head                            fp32 [V, H] matrix (hipBLASLt) or Int4Linear (quantize_lm_head)

Weights are seeded random (N(0, 0.02) linears and embedding, norms 1 + N(0, 0.1)); there are
no checkpoints on this path. The AWQ per-input-channel scales are searched (the reference's
``_search_awq_scale``) on synthetic calibration activations with 1% of channels scaled x20.
"""

from __future__ import annotations

import functools
from dataclasses import dataclass

import torch
from torch import nn

import ctypes

from .attention import paged_attention
from .kernels import load_fused_ops, load_paged_attention
from .quant import Int4Linear, _search_awq_scale


def _fused_ops():
    fo = load_fused_ops()
    if fo is None:
        raise RuntimeError("QuantCausalLM runs the fused HIP kernels of this package: build the "
                           "native library (llm-serving-engine_amd/build.py)")
    return fo


@functools.lru_cache(maxsize=None)
def _xfrag_splits(M: int, N: int, K: int) -> int:
    """K planes of the decode step's narrow linears (llmserve_int4_xfrag_splits)."""
    return int(_fused_ops().int4_xfrag_splits(M, N, K))


@dataclass
class ModelConfig:
    """The fields of the reference's ModelConfig (config.py:13-33) that the decode step uses;
    defaults are Qwen3-0.6B."""

    vocab_size: int = 151936
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    max_position_embeddings: int = 40960
    tie_word_embeddings: bool = True
    qk_norm: bool = True
    model_type: str = "qwen3"


QWEN3_0_6B = ModelConfig()


def rope_tables(head_dim: int, theta: float, max_positions: int) -> tuple[torch.Tensor, torch.Tensor]:
    """cos / sin [max_positions, head_dim] float32, built as RotaryEmbedding (models/layers.py:
    51-63, no scaling): inv_freq = 1 / theta^(2i/D), emb = [t * inv_freq, t * inv_freq] in
    float64, rounded to float32. Built once on the host at load time."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim))
    t = torch.arange(max_positions, dtype=torch.float64)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().float(), emb.sin().float()


class DecoderLayer(nn.Module):
    """One layer's weights: fp32 norms (buffers) and four Int4Linear submodules."""

    input_layernorm: torch.Tensor
    post_attention_layernorm: torch.Tensor
    q_norm: torch.Tensor | None
    k_norm: torch.Tensor | None
    qkv_proj: Int4Linear
    o_proj: Int4Linear
    gate_up_proj: Int4Linear
    down_proj: Int4Linear


class QuantCausalLM(nn.Module):
    """Random-init int4-AWQ model with fp32 embedding and norms, on one ROCm device."""

    def __init__(
        self,
        cfg: ModelConfig,
        group_size: int = 128,
        quantize_lm_head: bool = False,
        awq: bool = True,
        seed: int = 0,
        device: torch.device | str = "cuda",
        max_positions: int | None = None,
        calib_rows: int = 64,
    ) -> None:
        super().__init__()
        if cfg.num_attention_heads % cfg.num_key_value_heads:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")
        self.cfg = cfg
        self.group_size = group_size
        dev = torch.device(device)
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
        nq, nk, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim

        def calib(n_in: int) -> torch.Tensor:
            x = torch.randn(calib_rows, n_in, generator=g, device=dev)
            out = torch.randperm(n_in, generator=g, device=dev)[: max(1, n_in // 100)]
            x[:, out] *= 20
            return x

        def lin(n_out: int, n_in: int, w: torch.Tensor | None = None) -> Int4Linear:
            if w is None:
                w = torch.randn(n_out, n_in, generator=g, device=dev) * 0.02
            base = nn.Linear(n_in, n_out, bias=False, device="meta")
            base.weight = nn.Parameter(w, requires_grad=False)
            s = _search_awq_scale(w, calib(n_in), group_size) if awq else None
            return Int4Linear(base, group_size, s, device=dev)

        def norm(n: int) -> torch.Tensor:
            return 1 + 0.1 * torch.randn(n, generator=g, device=dev)

        self.layers = nn.ModuleList()
        for _ in range(cfg.num_hidden_layers):
            L = DecoderLayer()
            L.register_buffer("input_layernorm", norm(H))
            L.register_buffer("post_attention_layernorm", norm(H))
            L.register_buffer("q_norm", norm(D) if cfg.qk_norm else None)
            L.register_buffer("k_norm", norm(D) if cfg.qk_norm else None)
            L.qkv_proj = lin((nq + 2 * nk) * D, H)
            L.o_proj = lin(H, nq * D)
            L.gate_up_proj = lin(2 * I, H)
            L.down_proj = lin(H, I)
            self.layers.append(L)
        self.register_buffer("embed", torch.randn(V, H, generator=g, device=dev) * 0.02)
        self.register_buffer("norm", norm(H))
        if cfg.tie_word_embeddings:
            lm_w = self.embed
        else:
            lm_w = torch.randn(V, H, generator=g, device=dev) * 0.02
        self.lm_head: Int4Linear | None = lin(V, H, lm_w) if quantize_lm_head else None
        self.register_buffer("lm_weight", None if quantize_lm_head else lm_w)
        cos, sin = rope_tables(D, cfg.rope_theta, max_positions or min(cfg.max_position_embeddings, 32768))
        self.register_buffer("rope_cos", cos.to(dev))
        self.register_buffer("rope_sin", sin.to(dev))
        self.scale = D ** -0.5

    # Where the linears run the packed matrix-core kernel (above the GEMV's rows) the norms,
    # silu * up and the attention merge write the next linear's activation fragments directly
    # (its x * inv_act_scale and bf16 split fused in), and the linears run the packed
    # matrix-core kernel on them: one launch less per linear, same result bits.
    fuse_xfrag = True
    # With fragments, the fp32 LM head runs the split-bf16 matrix-core kernel
    # (lm_head_f32_xfrag: three bf16 pieces of each operand, every product fp32-faithful)
    # instead of torch.mm (hipBLASLt); at 1-4 rows the fp32 GEMV lm_head_f32 (exact fp32,
    # reads the matrix once at HBM speed).
    fp32_head_kernel = True

    # Up to chain_max_rows rows the step runs one persistent launch per layer for the whole
    # linear chain (o_proj .. next qkv, with the norms, silu * up, RoPE and the cache write:
    # llmserve_decode_chain) instead of a launch per op. The kernel takes up to 4 rows, but its
    # dot products run on ~160 CUs' VALUs, so its time grows with the rows: per Qwen3-0.6B
    # layer on MI355X, 19.5 us against 24.9 us per-op at 1 row, 26.2 / 27.5 at 2 and
    # 40.5 / 31.7 at 4.
    use_chain = True
    chain_max_rows = 2
    chain_spin_limit = 1 << 22  # polls per hand-off wait before the chain gives up

    def _chain_ok(self, rows: int) -> bool:
        cfg = self.cfg
        if not (self.use_chain and 1 <= rows <= 4 and self.embed.is_cuda):
            return False
        H, I, D = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
        heads = cfg.num_attention_heads + 2 * cfg.num_key_value_heads
        if D != 128 or self.group_size != 128 or cfg.num_attention_heads * D > 2048:
            return False
        if not (256 <= H <= 1024 and H % 128 == 0 and H % (2 * heads) == 0):
            return False
        if not (I % 512 == 0 and I <= 4096 and I % (H // 8) == 0):
            return False
        C = I // (H // 8)
        return (C % 8 == 0 and C <= 32 and cfg.num_attention_heads == 2 * cfg.num_key_value_heads
                and cfg.num_key_value_heads <= 8)

    @staticmethod
    def _chain_attn_ok(kv_layers, block_size: int, block_tables: torch.Tensor) -> bool:
        """The chain's fused attention: int8 caches addressable with 32-bit offsets, blocks of
        a power of two >= 8 tokens."""
        kc = kv_layers[0][0]
        if not (hasattr(kc, "scale") and kc.data.dtype == torch.int8):
            return False
        return (block_size >= 8 and block_size & (block_size - 1) == 0
                and kc.data.numel() < 2**32 and block_tables.shape[1] * block_size < 2**31)

    def chain_workspace(self) -> torch.Tensor:
        """The chain's hand-off workspace (zeroed once, then owned by the chain launches of
        this model: steps on one model must not overlap)."""
        ws = getattr(self, "_chain_ws", None)
        if ws is None:
            from ._native import capi

            n = capi().llmserve_decode_chain_workspace_bytes(self.cfg.hidden_size,
                                                             self.cfg.intermediate_size)
            ws = torch.zeros(n, dtype=torch.uint8, device=self.embed.device)
            self._chain_ws = ws
        return ws

    def chain_error(self) -> int:
        """Nonzero when a chain hand-off wait ran out of polls (synchronizes)."""
        from ._native import capi, check

        err = ctypes.c_int(0)
        check(capi().llmserve_decode_chain_error(ctypes.c_void_p(self.chain_workspace().data_ptr()),
                                                 ctypes.byref(err)))
        return err.value

    def check_chain(self) -> None:
        """Raises when a chain launch since the last check gave up on a hand-off wait (its
        workgroups then left rows of the step's outputs unwritten, so the step is invalid).
        Clears the error word first, so the next step starts clean. Synchronizes; a no-op when
        no chain step ran since the last check."""
        if not getattr(self, "_chain_pending", False):
            return
        self._chain_pending = False
        if self.chain_error():
            self.chain_workspace()[8:12].zero_()  # ctl[2], the error word (a fill kernel)
            raise RuntimeError("decode_chain: a hand-off wait ran out of polls (spin_limit "
                               f"{self.chain_spin_limit}); the step's outputs are invalid")

    def _chain(self, *, rows, x_out, q_in=None, attn_caches=None, x_in=None, ids=None,
               layer=None, nxt=None, h_out=None, q_out=None, caches=None, context_lens=None,
               block_tables=None, block_size=16, spin_limit=None) -> None:
        """One llmserve_decode_chain launch: layer ``layer``'s attention (of ``q_in`` over
        ``attn_caches``) and MLP half (None: embedding mode) and ``nxt``'s qkv part (None: the
        last layer, writing ``h_out``). ``q_out`` must not be ``q_in``."""
        from ._native import capi, check

        cfg = self.cfg

        def p(t):
            return None if t is None else ctypes.c_void_p(t.data_ptr())

        def lin(m):
            return [p(m.nibbles), p(m.g_scale), p(m.g_zero), p(m.inv_act_scale)] if m else [None] * 4

        ws = self.chain_workspace()
        kc = vc = None
        if nxt is not None:
            kc, vc = caches
        if layer is not None:
            ak, av = attn_caches
            args = [p(q_in), p(ak.data), p(av.data), p(ak.scale), p(av.scale), p(ak._q_mult),
                    ctypes.c_float(self.scale)]
            slots = ak.data.shape[0]
        else:
            args = [None] * 6 + [ctypes.c_float(self.scale)]
            slots = kc.data.shape[0]
        args += [p(x_in), p(ids), p(self.embed), cfg.vocab_size, p(x_out), p(h_out)]
        args += lin(layer.o_proj if layer else None)
        args += [p(layer.post_attention_layernorm) if layer else None]
        args += lin(layer.gate_up_proj if layer else None)
        args += lin(layer.down_proj if layer else None)
        args += [p(nxt.input_layernorm if nxt is not None else self.norm)]
        args += lin(nxt.qkv_proj if nxt is not None else None)
        args += [p(nxt.q_norm) if nxt is not None else None, p(nxt.k_norm) if nxt is not None else None,
                 p(self.rope_cos), p(self.rope_sin), self.rope_cos.shape[0], p(context_lens),
                 p(block_tables), block_tables.shape[1] if block_tables is not None else 0,
                 block_size, p(kc.smooth) if kc is not None else None, p(q_out),
                 p(kc.data) if kc is not None else None, p(vc.data) if vc is not None else None,
                 p(kc.scale) if kc is not None else None, p(vc.scale) if vc is not None else None,
                 slots, rows, cfg.hidden_size,
                 cfg.intermediate_size, cfg.num_attention_heads, cfg.num_key_value_heads,
                 cfg.head_dim, self.group_size, ctypes.c_float(cfg.rms_norm_eps), p(ws), ws.numel(),
                 self.chain_spin_limit if spin_limit is None else spin_limit,
                 ctypes.c_void_p(torch.cuda.current_stream(ws.device).cuda_stream)]
        check(capi().llmserve_decode_chain(*args))
        self._chain_pending = True

    def _forward_decode_chain(self, ids, context_lens, block_tables, kv_layers, block_size):
        """forward_decode for 1..4 rows: an embedding + layer-0 qkv launch, then one launch
        per layer for its attention, linear chain and the next layer's qkv (the last one
        writes the final norm's output)."""
        cfg = self.cfg
        B, H = ids.numel(), cfg.hidden_size
        nq, D = cfg.num_attention_heads, cfg.head_dim
        dev = self.embed.device
        n = len(self.layers)
        x = torch.empty(B, H, device=dev)
        q = torch.empty(B, nq, D, device=dev)
        self._chain(rows=B, x_out=x, ids=ids, nxt=self.layers[0], q_out=q, caches=kv_layers[0],
                    context_lens=context_lens, block_tables=block_tables, block_size=block_size)
        h = None
        for i, L in enumerate(self.layers):
            nxt = self.layers[i + 1] if i + 1 < n else None
            x_new = torch.empty(B, H, device=dev)
            q_new = torch.empty(B, nq, D, device=dev) if nxt is not None else None
            if nxt is None:
                h = torch.empty(B, H, device=dev)
            self._chain(rows=B, x_out=x_new, q_in=q, attn_caches=kv_layers[i], x_in=x, layer=L,
                        nxt=nxt, h_out=h, q_out=q_new,
                        caches=kv_layers[i + 1] if nxt is not None else None,
                        context_lens=context_lens, block_tables=block_tables,
                        block_size=block_size)
            x, q = x_new, q_new
        return h

    def _xfrag_ok(self, rows: int) -> bool:
        lins = [m for L in self.layers for m in (L.qkv_proj, L.o_proj, L.gate_up_proj, L.down_proj)]
        # the attention merge writes fragments of whole 128-channel blocks: head_dim 128 or 256
        return (self.fuse_xfrag and self.cfg.head_dim in (128, 256)
                and all(m.packed_path(rows) for m in lins))

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor, kv_caches,
                meta) -> torch.Tensor:
        """Final hidden states [T, H] of a ragged batch (prefill chunks and decode tokens laid
        end to end): the reference's calling convention and fused order (CausalLM.forward ->
        _forward_fused, models/transformer.py:128-190). ``positions`` [T] index the RoPE
        tables; ``kv_caches`` is ``KVCache.layers`` (int8 or fp32); ``meta`` the step's
        ``AttentionMetadata``. ``paged_attention`` writes this step's K/V and attends."""
        cfg = self.cfg
        fo = _fused_ops()
        nq, nk, D, eps = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.rms_norm_eps
        ids = input_ids.reshape(-1).to(device=self.embed.device, dtype=torch.long).contiguous()
        pos = positions.reshape(-1).to(device=self.embed.device, dtype=torch.long)
        T = ids.numel()
        cos = self.rope_cos.index_select(0, pos).contiguous()
        sin = self.rope_sin.index_select(0, pos).contiguous()
        x, h = fo.embed_rmsnorm(ids, self.embed, self.layers[0].input_layernorm, eps)
        n = len(self.layers)
        for i, (L, (kc, vc)) in enumerate(zip(self.layers, kv_caches, strict=True)):
            qkv = L.qkv_proj(h).contiguous()
            fo.rope_qk_(qkv, cos, sin, nq, nk, D, L.q_norm, L.k_norm, eps)
            q = qkv[:, : nq * D].view(T, nq, D)
            k = qkv[:, nq * D: (nq + nk) * D].view(T, nk, D)
            v = qkv[:, (nq + nk) * D:].view(T, nk, D)
            o = paged_attention(q, k, v, kc, vc, meta, self.scale)
            attn = L.o_proj(o.reshape(T, nq * D)).contiguous()
            h = fo.add_rmsnorm_(x, attn, L.post_attention_layernorm, eps)
            down = L.down_proj(fo.silu_mul(L.gate_up_proj(h).contiguous())).contiguous()
            nxt = self.layers[i + 1].input_layernorm if i + 1 < n else self.norm
            h = fo.add_rmsnorm_(x, down, nxt, eps)
        return h

    def forward_decode(self, ids: torch.Tensor, context_lens: torch.Tensor,
                       block_tables: torch.Tensor, kv_layers, block_size: int) -> torch.Tensor:
        """Final hidden states [B, H] of one decode token per sequence (or, when the int4 LM
        head consumes it, its activation fragments: ``compute_logits`` takes either).

        ``ids`` [B] int64; ``context_lens`` [B] int64 counts the token being decoded (its
        position is ctx - 1); ``block_tables`` [B, max_blocks] int64 holds the blocks of every
        position up to ctx - 1; ``kv_layers`` is ``KVCache.layers`` with int8 ``QuantizedKV``
        pairs. Writes this token's K and V into the caches. No host synchronization."""
        if (self._chain_ok(ids.numel()) and ids.numel() <= self.chain_max_rows
                and self._chain_attn_ok(kv_layers, block_size, block_tables)):
            return self._forward_decode_chain(ids, context_lens, block_tables, kv_layers,
                                              block_size)
        cfg = self.cfg
        fo, pa = _fused_ops(), load_paged_attention()
        nq, nk, D, eps = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.rms_norm_eps
        B, H, I = ids.shape[0], cfg.hidden_size, cfg.intermediate_size
        n = len(self.layers)
        frag = self._xfrag_ok(B)

        def gemm(xf, lin, K):
            return fo.int4_linear_gemm_xfrag(xf, lin.gemm_packed, B, lin.out_features, K,
                                             lin.group_size)

        def gemm_planes(xf, lin, K):
            """The linear before a residual norm: as K-split output planes [P, B, N] when its
            output alone would leave CUs idle (add_rmsnorm_xfrag_ adds them in order)."""
            P = _xfrag_splits(B, lin.out_features, K)
            if P == 1:
                return gemm(xf, lin, K)
            return fo.int4_linear_gemm_xfrag_split(xf, lin.gemm_packed, B, lin.out_features, K,
                                                   lin.group_size, P)

        if frag:
            x, h = fo.embed_rmsnorm_xfrag(ids, self.embed, self.layers[0].input_layernorm,
                                          self.layers[0].qkv_proj.inv_act_scale, eps)
        else:
            x, h = fo.embed_rmsnorm(ids, self.embed, self.layers[0].input_layernorm, eps)
        for i, (L, (kc, vc)) in enumerate(zip(self.layers, kv_layers, strict=True)):
            qkv = gemm(h, L.qkv_proj, H) if frag else L.qkv_proj(h)
            q = fo.decode_qkv_kv(qkv, self.rope_cos, self.rope_sin, context_lens, block_tables,
                                 block_size, L.q_norm, L.k_norm, eps, kc.smooth, kc.data, vc.data,
                                 kc.scale, vc.scale, nq, nk, D)
            if frag:  # the attention merge writes o_proj's input fragments
                _, xo = pa.paged_attention_decode_int8_xfrag(
                    q, kc.data, vc.data, kc.scale, vc.scale, block_tables, context_lens,
                    block_size, self.scale, 0, kc._q_mult, L.o_proj.inv_act_scale)
                attn = gemm_planes(xo, L.o_proj, nq * D)
            else:
                o = pa.paged_attention_decode_int8(q, kc.data, vc.data, kc.scale, vc.scale,
                                                   block_tables, context_lens, block_size,
                                                   self.scale, 0, kc._q_mult)
                attn = L.o_proj(o.view(B, nq * D))
            nxt = self.layers[i + 1] if i + 1 < n else None
            nxt_w = nxt.input_layernorm if nxt is not None else self.norm
            if frag:
                h = fo.add_rmsnorm_xfrag_(x, attn, L.post_attention_layernorm,
                                          L.gate_up_proj.inv_act_scale, eps)
                a = fo.silu_mul_xfrag(gemm(h, L.gate_up_proj, H), L.down_proj.inv_act_scale)
                to_frag = nxt is not None or self._lm_frag(B)
                down = gemm_planes(a, L.down_proj, I) if to_frag else gemm(a, L.down_proj, I)
                if nxt is not None:
                    h = fo.add_rmsnorm_xfrag_(x, down, nxt_w, nxt.qkv_proj.inv_act_scale, eps)
                elif self._lm_frag(B):
                    inv = self.lm_head.inv_act_scale if self.lm_head is not None else None
                    h = fo.add_rmsnorm_xfrag_(x, down, nxt_w, inv, eps)
                else:
                    h = fo.add_rmsnorm_(x, down, nxt_w, eps)
            else:
                h = fo.add_rmsnorm_(x, attn, L.post_attention_layernorm, eps)
                down = L.down_proj(fo.silu_mul(L.gate_up_proj(h)))
                h = fo.add_rmsnorm_(x, down, nxt_w, eps)
        return h

    def _lm_frag(self, rows: int) -> bool:
        """The LM head reads the final norm's activation fragments: the int4 head on its packed
        weight, or the fp32 head's split-bf16 matrix-core kernel (``fp32_head_kernel``)."""
        m = self.lm_head
        if not self._xfrag_ok(rows):
            return False
        if m is not None:
            return m.packed_path(rows)
        return self.fp32_head_kernel and self.cfg.hidden_size % 128 == 0

    def compute_logits(self, hidden: torch.Tensor, rows: int | None = None) -> torch.Tensor:
        """lm_head (transformer.py:192-193): fp32 [B, V]. ``hidden`` is the fp32 [B, H] final
        norm output, or (``rows`` given) the int4 LM head's activation fragments."""
        if rows is not None:
            m = self.lm_head
            if m is None:
                return load_fused_ops().lm_head_f32_xfrag(hidden, self.lm_weight, rows)
            return load_fused_ops().int4_linear_gemm_xfrag(hidden, m.gemm_packed, rows,
                                                           m.out_features, m.in_features,
                                                           m.group_size)
        if self.lm_head is not None:
            return self.lm_head(hidden)
        fo = load_fused_ops() if hidden.is_cuda else None
        if (fo is not None and self.fp32_head_kernel and 1 <= hidden.shape[0] <= 4
                and hidden.shape[1] in (256, 512, 1024)):
            return fo.lm_head_f32(hidden.contiguous(), self.lm_weight)  # exact fp32 GEMV
        return torch.mm(hidden, self.lm_weight.t())

    def weight_bytes(self, rows: int) -> dict[str, int]:
        """Bytes a decode step of ``rows`` tokens reads from the weights, by part: for each
        int4 linear the buffers its kernel at that batch reads (the reference-layout nibbles,
        scales and zeros for the GEMV, the packed copy for the matrix-core kernel) and the
        AWQ pre-scale; the fp32 LM head matrix."""

        def lin_bytes(m: Int4Linear) -> int:
            inv = 0 if m.inv_act_scale is None else m.inv_act_scale.numel() * 4
            if m.packed_path(rows):
                return m.gemm_packed.numel() + inv
            return (m.nibbles.numel() + (m.g_scale.numel() + m.g_zero.numel()) * 4) + inv

        lin = sum(lin_bytes(m) for L in self.layers
                  for m in (L.qkv_proj, L.o_proj, L.gate_up_proj, L.down_proj))
        lm = lin_bytes(self.lm_head) if self.lm_head is not None else self.lm_weight.numel() * 4
        return {"linears": lin, "lm_head": lm}
