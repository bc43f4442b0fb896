"""Native kernel loaders (reference: src/llmserve/kernels/__init__.py:19-72).

The reference JIT-compiles CPU extensions and each loader returns ``None`` when its build
fails, so that the callers fall back to PyTorch. Here the kernels are prebuilt gfx950 HIP code
(``llmserve/_lib``, built by ``llm-serving-engine_amd/build.py``); each loader returns a
namespace of ``torch.ops.llmserve_hip`` functions, or ``None`` with a logged warning when the
library is missing or does not load. The callers (``Int8Linear``, ``Int4Linear``,
``QuantizedKV``, ``paged_attention``) then compute with torch ops, as the reference's do; the
native functions take ROCm tensors only, so the callers also use torch for CPU tensors.

Functions, with the reference's names and signatures where the reference has them:

* ``load_int8_gemv()``: ``int8_linear(x, qweight, scale)`` and ``int4_linear(x, nibbles, scale,
  zero, group_size, inv_act_scale=None)`` (int8_gemv.cpp:109-112; ``inv_act_scale`` fuses
  Int4Linear's AWQ pre-scale); ``int8_linear_prefill(x, qweight, scale)``, Int8Linear's
  large-M path on the bf16 matrix cores (quant.py:71-72); ``int4_linear_gemm(...)``,
  Int4Linear's large-M path (quant.py:141-142); ``int4_gemm_pack(nibbles, scale, zero,
  group_size)`` and ``int4_linear_gemm_packed(x, packed, out_features, group_size,
  inv_act_scale=None)``, the decode-batch matrix-core kernel on a rearranged weight.
* ``load_paged_attention()``: ``paged_attention_decode_int8(q, k_cache, v_cache, k_scale,
  v_scale, block_tables, context_lens, block_size, scale, partition_size=0, q_mult=None)`` and
  ``paged_attention_decode(q, k_cache, v_cache, block_tables, context_lens, block_size, scale,
  partition_size=0)`` (fp32 cache) (paged_attention.cpp:386-399); ``paged_attention_rows``
  (every token of a ragged batch as one query row, decode and prefill alike) and
  ``attention_metadata`` (slots and query rows of a step, on the device).
* ``load_quant()``: the load-time quantizers and the int8 KV-cache write.
* ``load_fused_ops()``: ``rmsnorm``, ``add_rmsnorm_``, ``silu_mul``, ``rope_qk_``
  (fused_ops.cpp:129-137) and the decode-step kernels of this package (embedding + norm, the
  fused post-qkv KV write, greedy selection, the activation-fragment producers and consumers).

The reference's attention module also calls ``paged_attention_decode_v1``, ``set_simd`` and
``simd_available`` on the attention namespace (paged_attention.cpp:386-399) and imports
``decode_kernel`` and ``paged_attention_op`` from this module (attention.py:260-289); they are
provided with the same meaning: v1 is the fp32 decode as one context partition per sequence
(the reference's previous kernel, one work item per sequence and kv head), and there is no
CPU SIMD branch to switch (``simd_available()`` is False, ``set_simd`` accepts and ignores its
flag: the GPU kernel is the only code path).

Intra-package imports are relative, so the package also loads under another name (the
reference's process keeps its own ``llmserve``; its loaders import this one by path as
``llmserve_mi355x``).
"""

from __future__ import annotations

import functools
import logging
from types import SimpleNamespace

import os

import torch

from .._native import NativeLibraryMissing, ops

__all__ = ["NativeLibraryMissing", "decode_kernel", "load_fused_ops", "load_int8_gemv",
           "load_paged_attention", "load_quant", "native_available", "paged_attention_op"]

log = logging.getLogger(__name__)


def _namespace(what: str, names: tuple[str, ...], **extra) -> SimpleNamespace | None:
    try:
        o = ops()
    except (NativeLibraryMissing, OSError, RuntimeError) as e:
        log.warning("%s unavailable, using the PyTorch fallback: %s", what, e)
        return None
    return SimpleNamespace(**{n: getattr(o, n) for n in names}, **extra)


def _decode_v1(o):
    def paged_attention_decode_v1(q, k_cache, v_cache, block_tables, context_lens, block_size,
                                  scale):
        """The fp32 decode with one context partition per sequence (paged_attention.cpp's v1
        entry: no split-context merge)."""
        width = max(1, int(block_tables.shape[1]) * int(block_size))
        return o.paged_attention_decode(q, k_cache, v_cache, block_tables, context_lens,
                                        block_size, scale, width)

    return paged_attention_decode_v1


def _set_simd(on: bool) -> None:
    """The reference's switch of its AVX-512 branch; the GPU kernel has one code path."""
    bool(on)


def _simd_available() -> bool:
    return False


def native_available() -> bool:
    """True when the gfx950 op library loads in this process."""
    return load_quant() is not None


@functools.cache
def load_int8_gemv() -> SimpleNamespace | None:
    """Weight-only int8 / int4 matmuls (HIP, gfx950), or None."""
    return _namespace("int8/int4 GEMV kernels", (
        "int8_linear", "int4_linear", "int8_linear_prefill", "int4_linear_gemm",
        "int4_gemm_pack", "int4_linear_gemm_packed"))


@functools.cache
def load_paged_attention() -> SimpleNamespace | None:
    """Paged attention over int8 and fp32 KV caches (HIP, gfx950), or None."""
    try:
        v1 = _decode_v1(ops())
    except (NativeLibraryMissing, OSError, RuntimeError):
        v1 = None
    return _namespace("paged attention kernels", (
        "paged_attention_decode_int8", "paged_attention_decode_int8_xfrag",
        "paged_attention_decode", "paged_attention_rows", "attention_metadata"),
        paged_attention_decode_v1=v1, set_simd=_set_simd, simd_available=_simd_available)


def decode_kernel():
    """The fp32 decode entry (reference kernels/__init__.py:75-81): ``paged_attention_decode``,
    or ``paged_attention_decode_v1`` when ``LLMSERVE_ATTN_KERNEL=v1``."""
    m = load_paged_attention()
    if os.environ.get("LLMSERVE_ATTN_KERNEL") == "v1":
        return m.paged_attention_decode_v1
    return m.paged_attention_decode


@functools.cache
def paged_attention_op():
    """``torch.ops.llmserve.paged_attention_decode`` (reference kernels/__init__.py:84-111): the
    fp32 decode as a custom op with a fake (shape-only) kernel, so ``torch.compile`` traces
    around it. When the reference's own module registered the op already in this process,
    that registration is returned."""
    try:
        @torch.library.custom_op("llmserve::paged_attention_decode", mutates_args=())
        def paged_attention_decode(q: torch.Tensor, k_cache: torch.Tensor,
                                   v_cache: torch.Tensor, block_tables: torch.Tensor,
                                   context_lens: torch.Tensor, block_size: int,
                                   scale: float) -> torch.Tensor:
            return decode_kernel()(q.contiguous(), k_cache, v_cache, block_tables, context_lens,
                                   block_size, scale)
    except RuntimeError:  # already defined by the reference's kernels module
        return torch.ops.llmserve.paged_attention_decode

    @paged_attention_decode.register_fake
    def _(q, k_cache, v_cache, block_tables, context_lens, block_size, scale):
        return torch.empty_like(q)

    return paged_attention_decode


@functools.cache
def load_quant() -> SimpleNamespace | None:
    """Load-time quantizers and the int8 KV-cache write (HIP, gfx950), or None."""
    return _namespace("quantization kernels", ("int8_quantize", "int4_quantize",
                                               "kv_quantize_write"))


@functools.cache
def load_fused_ops() -> SimpleNamespace | None:
    """Decoder-layer elementwise ops and decode-step glue (HIP, gfx950), or None."""
    return _namespace("fused ops", (
        "rmsnorm", "add_rmsnorm_", "embed_rmsnorm", "add_rmsnorm_xfrag_", "embed_rmsnorm_xfrag",
        "silu_mul_xfrag", "int4_linear_gemm_xfrag", "int4_linear_gemm_xfrag_split",
        "int4_xfrag_splits", "lm_head_f32_xfrag", "lm_head_f32",
        "silu_mul", "rope_qk_", "decode_qkv_kv", "argmax_advance"))
