"""ORACLE (test infrastructure only) — numpy/ctypes front end of the C restatement
(oracle/cpu_kernels.c) and loader of the reference's own compiled kernels (oracle/_ref/).

Pinned by tests/test_oracle_cpu.py (float64 mathematics; the reference's kernels when built).
"""

from __future__ import annotations

import ctypes
import functools
import importlib.machinery
import importlib.util
from pathlib import Path

import numpy as np

from oracle.build import ISAS, cpu_lib_path, ref_module_path

_P, _I64, _F32, _I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int


def host_isa() -> str:
    """Highest ISA level of oracle/build.py's list that this CPU runs."""
    flags: set[str] = set()
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("flags"):
                flags = set(line.split(":", 1)[1].split())
                break
    except OSError:
        pass
    v4 = {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"}
    v3 = {"avx2", "fma", "bmi1", "bmi2", "movbe"}
    if v4 <= flags and v3 <= flags:
        return "x86-64-v4"
    if v3 <= flags:
        return "x86-64-v3"
    raise RuntimeError("oracle CPU libraries need at least x86-64-v3 (AVX2/FMA)")


@functools.cache
def lib(isa: str | None = None) -> ctypes.CDLL:
    isa = isa or host_isa()
    path = cpu_lib_path(isa)
    if not path.is_file():
        raise FileNotFoundError(f"{path} not built (python oracle/build.py)")
    L = ctypes.CDLL(str(path))
    L.oracle_int8_linear.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64]
    L.oracle_int8_linear.restype = None
    L.oracle_int4_linear.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64]
    L.oracle_int4_linear.restype = None
    L.oracle_paged_decode_int8.argtypes = [_P] * 8 + [_I64] * 6 + [_F32, _I64]
    L.oracle_paged_decode_int8.restype = _I64
    L.oracle_set_threads.argtypes = [_I32]
    L.oracle_set_threads.restype = None
    L.oracle_get_threads.argtypes = []
    L.oracle_get_threads.restype = _I32
    return L


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


def get_threads() -> int:
    return int(lib().oracle_get_threads())


def int8_linear(x: np.ndarray, q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    q = np.ascontiguousarray(q, np.int8)
    scale = np.ascontiguousarray(scale, np.float32)
    M, K = x.shape
    N = q.shape[0]
    assert q.shape[1] == K and M <= 64
    y = np.empty((M, N), np.float32)
    lib().oracle_int8_linear(_ptr(x), _ptr(q), _ptr(scale), _ptr(y), M, N, K)
    return y


def int4_linear(x, nib, g_scale, g_zero, group_size, inv_act_scale=None) -> np.ndarray:
    """Int4Linear.forward's small-batch path: x * inv_act_scale (float32), then int4_linear."""
    x = np.ascontiguousarray(x, np.float32)
    if inv_act_scale is not None:
        x = np.ascontiguousarray((x * inv_act_scale[None, :]).astype(np.float32))
    nib = np.ascontiguousarray(nib, np.uint8)
    g_scale = np.ascontiguousarray(g_scale, np.float32)
    g_zero = np.ascontiguousarray(g_zero, np.float32)
    M, K = x.shape
    N = nib.shape[0]
    assert nib.shape[1] * 2 == K and K % group_size == 0 and group_size % 2 == 0 and M <= 64
    y = np.empty((M, N), np.float32)
    lib().oracle_int4_linear(_ptr(x), _ptr(nib), _ptr(g_scale), _ptr(g_zero), _ptr(y), M, N, K,
                             group_size)
    return y


def paged_decode_int8(q, k_cache, v_cache, k_scale, v_scale, block_tables, context_lens,
                      block_size, scale, partition_size=0, q_mult=None) -> np.ndarray:
    """paged_attention_decode_int8 with the q * q_mult smoothing product applied first."""
    q = np.ascontiguousarray(q, np.float32)
    if q_mult is not None:
        q = np.ascontiguousarray((q * q_mult[None]).astype(np.float32))
    k_cache = np.ascontiguousarray(k_cache, np.int8)
    v_cache = np.ascontiguousarray(v_cache, np.int8)
    k_scale = np.ascontiguousarray(k_scale, np.float32)
    v_scale = np.ascontiguousarray(v_scale, np.float32)
    bt = np.ascontiguousarray(block_tables, np.int64)
    cl = np.ascontiguousarray(context_lens, np.int64)
    B, Hq, D = q.shape
    Hk = k_cache.shape[1]
    out = np.empty_like(q)
    rc = lib().oracle_paged_decode_int8(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale),
                                        _ptr(v_scale), _ptr(bt), _ptr(cl), _ptr(out), B, Hq, Hk,
                                        D, bt.shape[1], block_size, float(scale), partition_size)
    if rc < 0:
        raise ValueError("oracle_paged_decode_int8: bad arguments")
    return out


def ref_available(isa: str | None = None) -> bool:
    try:
        isa = isa or host_isa()
    except RuntimeError:
        return False
    return all(ref_module_path(isa, n).is_file()
               for n in ("llmserve_int8_gemv", "llmserve_paged_attention", "llmserve_fused_ops"))


@functools.cache
def ref_module(name: str, isa: str | None = None):
    """The reference's compiled kernel module ``name`` (llmserve_int8_gemv,
    llmserve_paged_attention or llmserve_fused_ops) from oracle/_ref/<isa>/. Needs torch
    (CPU tensors)."""
    import torch  # noqa: F401  (the extension links libtorch)

    isa = isa or host_isa()
    path = ref_module_path(isa, name)
    if not path.is_file():
        raise FileNotFoundError(f"{path} not built (python oracle/build.py with the reference)")
    loader = importlib.machinery.ExtensionFileLoader(name, str(path))
    spec = importlib.util.spec_from_file_location(name, str(path), loader=loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    return mod


__all__ = ["ISAS", "host_isa", "int4_linear", "int8_linear", "lib", "paged_decode_int8",
           "ref_available", "ref_module", "set_threads", "get_threads"]
