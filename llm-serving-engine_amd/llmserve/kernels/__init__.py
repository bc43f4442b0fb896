"""Native kernel loaders (reference: src/llmserve/kernels/__init__.py:19-72).

The reference JIT-compiles three CPU extensions and returns ``None`` when a build fails, so
that callers fall back to PyTorch. Here the kernels are prebuilt gfx950 HIP code and there is
no fallback: a missing library raises ``NativeLibraryMissing`` (a RuntimeError). The returned
objects expose the reference's function names and signatures:

* ``load_int8_gemv()``: ``int8_linear(x, qweight, scale)`` and
  ``int4_linear(x, nibbles, scale, zero, group_size, inv_act_scale=None)``
  (int8_gemv.cpp:109-112; ``inv_act_scale`` fuses Int4Linear's AWQ pre-scale), and
  ``int8_linear_prefill(x, qweight, scale)``: Int8Linear's large-M path on the bf16 matrix
  cores (quant.py:71-72), and ``int4_linear_gemm(x, nibbles, scale, zero, group_size,
  inv_act_scale=None)``: Int4Linear's large-M path (quant.py:141-142) on the matrix cores;
  ``int4_gemm_pack(nibbles, scale, zero, group_size)`` rearranges an int4 weight once for
  ``int4_linear_gemm_packed(x, packed, out_features, group_size, inv_act_scale=None)``, the
  same product with the decode-batch matrix-core kernel;
* ``load_paged_attention()``: ``paged_attention_decode_int8(q, k_cache, v_cache, k_scale,
  v_scale, block_tables, context_lens, block_size, scale, partition_size=0, q_mult=None)``
  (paged_attention.cpp:386-399; ``q_mult`` fuses the key-smoothing multiply of q).

* ``load_fused_ops()``: ``rmsnorm(x, w, eps)``, ``add_rmsnorm_(x, r, w, eps)``,
  ``silu_mul(gate_up)`` and ``rope_qk_(qkv, cos, sin, n_q, n_k, head_dim, q_w=None, k_w=None,
  eps=1e-6)`` (fused_ops.cpp:129-137), plus the decode-step glue ``embed_rmsnorm(ids, embed,
  w, eps) -> (x, h)`` (embedding lookup + first input norm), ``decode_qkv_kv`` (q/k norm,
  RoPE and the int8 KV-cache write in one launch) and ``argmax_advance`` (greedy next token);
  and the producers of the packed int4 linear's activation fragments, which fuse the next
  linear's ``x * inv_act_scale`` and bf16 split into the norm / silu kernel:
  ``add_rmsnorm_xfrag_(x, r, w, act_inv, eps)``, ``embed_rmsnorm_xfrag(ids, embed, w, act_inv,
  eps) -> (x, xfrag)``, ``silu_mul_xfrag(gate_up, act_inv)``, consumed by
  ``int4_linear_gemm_xfrag(xfrag, packed, M, N, K, group_size)``.

The fp32-KV decode variants (``paged_attention_decode``, ``paged_attention_decode_v1``,
``set_simd``) are outside the quantized path and not provided.
"""

from __future__ import annotations

import functools
from types import SimpleNamespace

from llmserve._native import NativeLibraryMissing, ops

__all__ = ["NativeLibraryMissing", "load_fused_ops", "load_int8_gemv", "load_paged_attention",
           "load_quant"]


@functools.cache
def load_int8_gemv() -> SimpleNamespace:
    """Weight-only int8 / int4 small-batch matmuls (HIP, gfx950)."""
    o = ops()
    return SimpleNamespace(int8_linear=o.int8_linear, int4_linear=o.int4_linear,
                           int8_linear_prefill=o.int8_linear_prefill,
                           int4_linear_gemm=o.int4_linear_gemm,
                           int4_gemm_pack=o.int4_gemm_pack,
                           int4_linear_gemm_packed=o.int4_linear_gemm_packed)


@functools.cache
def load_paged_attention() -> SimpleNamespace:
    """int8-KV paged decode attention (HIP, gfx950)."""
    o = ops()
    return SimpleNamespace(paged_attention_decode_int8=o.paged_attention_decode_int8,
                           paged_attention_decode_int8_xfrag=o.paged_attention_decode_int8_xfrag)


@functools.cache
def load_quant() -> SimpleNamespace:
    """Load-time quantizers and the int8 KV-cache write (HIP, gfx950)."""
    o = ops()
    return SimpleNamespace(
        int8_quantize=o.int8_quantize,
        int4_quantize=o.int4_quantize,
        kv_quantize_write=o.kv_quantize_write,
    )


@functools.cache
def load_fused_ops() -> SimpleNamespace:
    """Decoder-layer elementwise ops and decode-step glue (HIP, gfx950)."""
    o = ops()
    return SimpleNamespace(
        rmsnorm=o.rmsnorm,
        add_rmsnorm_=o.add_rmsnorm_,
        embed_rmsnorm=o.embed_rmsnorm,
        add_rmsnorm_xfrag_=o.add_rmsnorm_xfrag_,
        embed_rmsnorm_xfrag=o.embed_rmsnorm_xfrag,
        silu_mul_xfrag=o.silu_mul_xfrag,
        int4_linear_gemm_xfrag=o.int4_linear_gemm_xfrag,
        lm_head_f32_xfrag=o.lm_head_f32_xfrag,
        silu_mul=o.silu_mul,
        rope_qk_=o.rope_qk_,
        decode_qkv_kv=o.decode_qkv_kv,
        argmax_advance=o.argmax_advance,
    )
