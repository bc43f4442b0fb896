"""ORACLE (test infrastructure only) — numpy restatement of the reference's quantizers.

All arithmetic is float32 with numpy's IEEE operations, matching torch's CPU elementwise ops
one operation at a time: true division, round-half-to-even (``np.rint`` = ``torch.round``),
no fused multiply-add. Pinned by tests/test_oracle_quant.py against torch-CPU golden vectors
(tests/golden/quant_golden.npz), hand-built tie and special cases, and the |deq - w| <= scale/2
round-trip bound.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def int8_quantize(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Int8Linear.__init__ (reference quant.py:41-43).

    scale = clamp_min(amax_k |w| / 127, 1e-8);  q = clamp(round(w / scale), -127, 127).
    """
    w = np.asarray(w, dtype=F32)
    amax = np.abs(w).max(axis=1)
    scale = np.maximum(amax / F32(127.0), F32(1e-8)).astype(F32)
    q = np.clip(np.rint(w / scale[:, None]), -127, 127).astype(np.int8)
    return q, scale


def int8_dequantize(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Int8Linear.dequantize (reference quant.py:78-79): q * scale[:, None] in float32."""
    return (q.astype(F32) * scale[:, None]).astype(F32)


def awq_fold(w: np.ndarray, act_scale: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """AWQ fold (reference quant.py:103-105): W * s[None, :] and inv_act_scale = 1 / s.

    torch evaluates ``1.0 / s`` as ``s.reciprocal() * 1.0``: one IEEE division.
    """
    w = np.asarray(w, dtype=F32)
    s = np.asarray(act_scale, dtype=F32)
    return (w * s[None, :]).astype(F32), (F32(1.0) / s).astype(F32)


def int4_quantize(w: np.ndarray, group_size: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """_int4_quantize (reference quant.py:82-90).

    Per group: mn, mx;  scale = clamp_min((mx - mn) / 15, 1e-8);
    q = clamp(round((w - mn) / scale), 0, 15);  zero = mn + 8 * scale.
    Returns q int32 [N, K], scale [N, G], zero [N, G].
    """
    w = np.asarray(w, dtype=F32)
    n, k = w.shape
    if k % group_size:
        raise ValueError(f"in_features {k} not divisible by group {group_size}")
    g = w.reshape(n, k // group_size, group_size)
    mn = g.min(-1, keepdims=True)
    mx = g.max(-1, keepdims=True)
    scale = np.maximum((mx - mn) / F32(15.0), F32(1e-8)).astype(F32)
    q = np.clip(np.rint((g - mn) / scale), 0, 15).astype(np.int32).reshape(n, k)
    zero = (mn + (F32(8.0) * scale).astype(F32)).astype(F32)
    return q, scale[..., 0], zero[..., 0]


def pack_nibbles(q: np.ndarray) -> np.ndarray:
    """Nibble packing (reference quant.py:113-114): byte j = q[2j] | q[2j+1] << 4."""
    q8 = q.astype(np.uint8)
    return (q8[:, 0::2] | (q8[:, 1::2] << 4)).astype(np.uint8)


def unpack_nibbles(nib: np.ndarray) -> np.ndarray:
    lo = (nib & 0xF).astype(np.int32)
    hi = (nib >> 4).astype(np.int32)
    return np.stack([lo, hi], axis=-1).reshape(nib.shape[0], -1)


def int4_dequantize(nib: np.ndarray, scale: np.ndarray, zero: np.ndarray, group_size: int) -> np.ndarray:
    """Int4Linear.dequantize (reference quant.py:126-132): (q - 8) * s + z in float32."""
    q = unpack_nibbles(nib).astype(F32)
    n, k = q.shape
    qg = q.reshape(n, k // group_size, group_size)
    w = ((qg - F32(8.0)) * scale[..., None]).astype(F32) + zero[..., None]
    return w.astype(F32).reshape(n, k)


def int4_quantize_pack(w: np.ndarray, group_size: int, act_scale: np.ndarray | None = None):
    """Int4Linear.__init__ buffers (reference quant.py:94-121):
    (nibbles uint8 [N, K/2], g_scale [N, G], g_zero [N, G], inv_act_scale [K] or None)."""
    inv = None
    if act_scale is not None:
        w, inv = awq_fold(w, act_scale)
    q, s, z = int4_quantize(w, group_size)
    return pack_nibbles(q), s, z, inv


def kv_quantize(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """QuantizedKV.quantize (reference attention.py:153-157): clamp, then divide.

    s = clamp_min(amax_d |x|, 1e-8) / 127;  q = clamp(round(x / s), -127, 127).
    """
    x = np.asarray(x, dtype=F32)
    s = (np.maximum(np.abs(x).max(-1), F32(1e-8)) / F32(127.0)).astype(F32)
    q = np.clip(np.rint(x / s[..., None]), -127, 127).astype(np.int8)
    return q, s


def kv_smooth(k: np.ndarray, smooth: np.ndarray) -> np.ndarray:
    """Key smoothing before the write (reference attention.py:245): k / s, IEEE division."""
    return (np.asarray(k, dtype=F32) / np.asarray(smooth, dtype=F32)).astype(F32)


def q_smooth(q: np.ndarray, q_mult: np.ndarray) -> np.ndarray:
    """Query side of the smoothing (reference attention.py:244): q * s repeated per GQA group."""
    return (np.asarray(q, dtype=F32) * np.asarray(q_mult, dtype=F32)).astype(F32)


def smoothing_from_stats(max_abs_k: np.ndarray, alpha: float) -> np.ndarray:
    """calibrate_k_smoothing's transform (reference attention.py:196-200):
    s = clamp_min(max|K|, 1e-5) ** alpha, divided by its mean over head_dim."""
    s = np.power(np.maximum(max_abs_k.astype(F32), F32(1e-5)), F32(alpha)).astype(F32)
    return (s / s.mean(-1, keepdims=True, dtype=F32)).astype(F32)


def awq_search_scale(w: np.ndarray, x: np.ndarray, group_size: int) -> tuple[np.ndarray, float]:
    """_search_awq_scale (reference quant.py:154-170) in float64 for the GEMMs: returns the
    scale vector and the chosen alpha. The candidate scales themselves are float32 as in the
    reference; only the error metric is evaluated in float64, which is what the grid choice
    depends on (ties closer than float32 GEMM rounding are unpinned)."""
    w = np.asarray(w, dtype=F32)
    x = np.asarray(x, dtype=F32)
    act = np.maximum(np.abs(x).mean(0, dtype=F32), F32(1e-5)).astype(F32)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    best, best_s, best_a = np.inf, None, None
    for i in range(11):
        alpha = i / 10
        s = np.power(act, F32(alpha)).astype(F32)
        s = (s / np.sqrt(s.max() * s.min()).astype(F32)).astype(F32)
        q, sc, z = int4_quantize((w * s[None, :]).astype(F32), group_size)
        deq = ((q.astype(F32).reshape(w.shape[0], -1, group_size) - F32(8)) * sc[..., None]
               + z[..., None]).reshape(w.shape).astype(F32)
        deq = (deq / s[None, :]).astype(F32)
        err = float(np.mean((x.astype(np.float64) @ deq.astype(np.float64).T - ref) ** 2))
        if err < best:
            best, best_s, best_a = err, s, alpha
    return best_s, best_a
