"""Loading of the in-tree gfx950 libraries.

``ops()`` registers ``torch.ops.llmserve_hip.*`` (``libllmserve_torch.so``) and ``capi()``
returns a ctypes handle on the C ABI of ``include/llmserve_hip.h`` (``libllmserve_hip.so``).
Both raise ``NativeLibraryMissing`` when the libraries were not built: the quantized path
has no CPU or PyTorch substitute, so a missing build must fail loudly rather than run
something else.
"""

from __future__ import annotations

import ctypes
import functools
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "_lib"
HIP_LIB = LIB_DIR / "libllmserve_hip.so"
TORCH_LIB = LIB_DIR / "libllmserve_torch.so"


class NativeLibraryMissing(RuntimeError):
    pass


def _require(path: Path) -> Path:
    if not path.is_file():
        raise NativeLibraryMissing(
            f"{path.name} is not built; run `python llm-serving-engine_amd/build.py` "
            "(or __graft_entry__.build()) first"
        )
    return path


@functools.cache
def ops():
    """The ``torch.ops.llmserve_hip`` namespace (loads the op library once)."""
    import torch

    torch.ops.load_library(str(_require(TORCH_LIB)))
    return torch.ops.llmserve_hip


# C ABI signatures, in the order of include/llmserve_hip.h.
_P, _I64, _I32, _F32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
C_SIGNATURES: dict[str, tuple[object, list]] = {
    "llmserve_last_error": (ctypes.c_char_p, []),
    "llmserve_abi_version": (_I32, []),
    "llmserve_time_next_call": (_I32, [_P, _P]),
    "llmserve_int8_quantize": (_I32, [_P, _P, _P, _I64, _I64, _P]),
    "llmserve_int4_quantize": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "llmserve_kv_quantize_write": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "llmserve_int8_linear": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "llmserve_int4_linear": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "llmserve_int4_linear_gemm_workspace_bytes": (_I64, [_I64, _I64]),
    "llmserve_int4_linear_gemm": (_I32, [_P] * 6 + [_I64] * 4 + [_P, _I64, _P]),
    "llmserve_int4_gemm_pack_bytes": (_I64, [_I64, _I64, _I64]),
    "llmserve_int4_gemm_pack": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P, _I64, _P]),
    "llmserve_int4_linear_gemm_packed_workspace_bytes": (_I64, [_I64, _I64]),
    "llmserve_int4_linear_gemm_packed": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P]),
    "llmserve_int4_xfrag_bytes": (_I64, [_I64, _I64]),
    "llmserve_int4_xfrag_split": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "llmserve_int4_linear_gemm_xfrag": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "llmserve_int4_xfrag_splits": (_I64, [_I64, _I64, _I64]),
    "llmserve_int4_packed_splits": (_I64, [_I64, _I64, _I64]),
    "llmserve_int4_linear_gemm_xfrag_split": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P]),
    "llmserve_rmsnorm_xfrag": (_I32, [_P, _P, _P, _P, _I64, _I64, _F32, _P]),
    "llmserve_add_rmsnorm_xfrag": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _F32, _P]),
    "llmserve_add_rmsnorm_split_xfrag": (_I32, [_P, _P, _I64, _P, _P, _P, _I64, _I64, _F32, _P]),
    "llmserve_embed_rmsnorm_xfrag": (_I32, [_P, _P, _I64, _P, _P, _P, _P, _I64, _I64, _F32, _P]),
    "llmserve_silu_mul_xfrag": (_I32, [_P, _P, _P, _I64, _I64, _P]),
    "llmserve_int8_linear_prefill_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "llmserve_int8_linear_prefill": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _P]),
    "llmserve_rmsnorm": (_I32, [_P, _P, _P, _I64, _I64, _F32, _P]),
    "llmserve_add_rmsnorm": (_I32, [_P, _P, _P, _P, _I64, _I64, _F32, _P]),
    "llmserve_embed_rmsnorm": (_I32, [_P, _P, _I64, _P, _P, _P, _I64, _I64, _F32, _P]),
    "llmserve_silu_mul": (_I32, [_P, _P, _I64, _I64, _P]),
    "llmserve_rope_qk": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _F32, _P]),
    "llmserve_decode_qkv_kv": (
        _I32,
        [_P, _I64, _P, _P, _I64, _P, _P, _I64, _I64, _P, _P, _F32, _P, _P, _P, _P, _P, _P]
        + [_I64] * 5 + [_P],
    ),
    "llmserve_argmax_advance_workspace_bytes": (_I64, [_I64]),
    "llmserve_argmax_advance": (_I32, [_P, _I64, _I64, _P, _P, _P, _I64, _P]),
    "llmserve_lm_head_f32_xfrag": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "llmserve_paged_attention_workspace_bytes": (_I64, [_I64] * 7),
    "llmserve_paged_attention_decode_int8": (
        _I32,
        [_P] * 8 + [_I64] * 7 + [_F32, _I64, _P, _P, _I64, _P],
    ),
    "llmserve_paged_attention_decode_int8_xfrag": (
        _I32,
        [_P] * 10 + [_I64] * 7 + [_F32, _I64, _P, _P, _I64, _P],
    ),
    "llmserve_paged_attention_decode": (_I32, [_P] * 6 + [_I64] * 7 + [_F32, _I64, _P, _I64, _P]),
    "llmserve_paged_attention_rows_int8": (
        _I32,
        [_P] * 6 + [_I64] + [_P] * 3 + [_I64] * 7 + [_F32, _P, _P, _I64, _P],
    ),
    "llmserve_paged_attention_rows_f32": (
        _I32,
        [_P] * 4 + [_I64] + [_P] * 3 + [_I64] * 7 + [_F32, _P, _P, _I64, _P],
    ),
    "llmserve_attention_metadata": (_I32, [_P, _P] + [_I64] * 4 + [_P] * 4),
    "llmserve_decode_chain_workspace_bytes": (_I64, [_I64, _I64]),
    "llmserve_decode_chain": (
        _I32,
        # q_in, this layer's caches and scales, q_mult, scale; x_in, ids, embed, vocab, x_out,
        # h_out; 22 weight / norm / RoPE pointers; max_pos, context_lens, block_tables,
        # max_blocks, block_size, k_smooth, q_out, the next layer's caches and scales,
        # num_slots; M, H, I, n_q, n_k, head_dim, group_size; eps, workspace, workspace_bytes,
        # spin_limit, stream
        [_P] * 6 + [_F32] + [_P, _P, _P, _I64, _P, _P] + [_P] * 22
        + [_I64, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64] + [_I64] * 7
        + [_F32, _P, _I64, _I64, _P],
    ),
    "llmserve_decode_chain_error": (_I32, [_P, _P]),
    "llmserve_paged_attention_noalloc_scratch_bytes": (_I64, []),
    "llmserve_paged_attention_decode_int8_noalloc": (
        _I32,
        [_P] * 8 + [_I64] * 7 + [_F32, _I64, _P, _P],
    ),
    "llmserve_sample": (_I32, [_P, _I64, _I64] + [_P] * 19 + [_I32, _I32, _P, _P]),
    "llmserve_lm_head_f32": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P]),
}


@functools.cache
def capi() -> ctypes.CDLL:
    """ctypes handle on libllmserve_hip.so with argument/return types set.

    In a process that uses torch, import torch first so that the library binds to the HIP
    runtime torch already loaded (both carry the SONAME libamdhip64.so.7).
    """
    lib = ctypes.CDLL(str(_require(HIP_LIB)))
    for name, (res, args) in C_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def check(rc: int) -> None:
    """Raises RuntimeError with the library's message for a nonzero C ABI status."""
    if rc != 0:
        raise RuntimeError(capi().llmserve_last_error().decode())


@functools.cache
def _hip_runtime() -> ctypes.CDLL:
    """The HIP runtime already loaded in this process (torch's; SONAME libamdhip64.so.7)."""
    import torch  # noqa: F401  (makes sure torch's runtime is the one bound)

    lib = ctypes.CDLL("libamdhip64.so.7")
    lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    lib.hipEventCreate.restype = ctypes.c_int
    lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), _P, _P]
    lib.hipEventElapsedTime.restype = ctypes.c_int
    lib.hipEventSynchronize.argtypes = [_P]
    lib.hipEventSynchronize.restype = ctypes.c_int
    lib.hipEventDestroy.argtypes = [_P]
    lib.hipEventDestroy.restype = ctypes.c_int
    return lib


class KernelTimer:
    """Kernel-execution time of single library calls: ``arm(i)`` makes the next call on this
    thread record event pair i around its kernels (llmserve_time_next_call), ``elapsed_ms(i)``
    reads it after the call."""

    def __init__(self, n: int) -> None:
        hip = _hip_runtime()
        self._ev = []
        for _ in range(2 * n):
            e = ctypes.c_void_p()
            if hip.hipEventCreate(ctypes.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")
            self._ev.append(e)

    def arm(self, i: int) -> None:
        check(capi().llmserve_time_next_call(self._ev[2 * i], self._ev[2 * i + 1]))

    def elapsed_ms(self, i: int) -> float:
        hip = _hip_runtime()
        hip.hipEventSynchronize(self._ev[2 * i + 1])
        ms = ctypes.c_float()
        if hip.hipEventElapsedTime(ctypes.byref(ms), self._ev[2 * i], self._ev[2 * i + 1]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def __del__(self) -> None:
        try:
            hip = _hip_runtime()
            for e in self._ev:
                hip.hipEventDestroy(e)
        except Exception:
            pass
