"""ORACLE (test infrastructure only) — numpy restatement of the reference's fused decoder-layer
ops (src/llmserve/kernels/csrc/fused_ops.cpp) and float64 references of the same mathematics.

float32 functions follow fused_ops.cpp operation by operation (order of the multiplies, the
clamp-free norm, the rotate-half RoPE); the reference compiles with -ffast-math, so its sums
may be reassociated and its multiply-adds fused: they agree with these to a few float32 ulps.

Pinned by tests/test_oracle_fused.py: against the reference's own compiled fused_ops
(tests/golden/fused_golden.npz, written by tests/golden/make_golden.py from oracle/_ref),
against the float64 mathematics, and by closed forms (a constant row normalizes to
sign * w; RoPE at position 0 is the identity; RoPE preserves the norm of every pair).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """fused_ops.cpp:23-30 (norm_row) per row of the last axis:
    inv = 1 / sqrt(sum(x^2) / H + eps); out = w * (x * inv)."""
    x = np.asarray(x, F32)
    H = x.shape[-1]
    ss = np.sum(x * x, axis=-1, dtype=F32, keepdims=True)
    inv = F32(1) / np.sqrt(ss / F32(H) + F32(eps))
    return (np.asarray(w, F32) * (x * inv)).astype(F32)


def add_rmsnorm(x: np.ndarray, r: np.ndarray, w: np.ndarray, eps: float):
    """fused_ops.cpp:58-81: x += r, then rmsnorm(x) * w. Returns (new x, out)."""
    x2 = (np.asarray(x, F32) + np.asarray(r, F32)).astype(F32)
    return x2, rmsnorm(x2, w, eps)


def silu_mul(gate_up: np.ndarray) -> np.ndarray:
    """fused_ops.cpp:83-99: out = g / (1 + exp(-g)) * u for a [T, 2I] gate|up row."""
    gu = np.asarray(gate_up, F32)
    I = gu.shape[-1] // 2
    g, u = gu[..., :I], gu[..., I:]
    return (g / (F32(1) + np.exp(-g)) * u).astype(F32)


def rope_qk(qkv: np.ndarray, cos: np.ndarray, sin: np.ndarray, n_q: int, n_k: int, D: int,
            q_w=None, k_w=None, eps: float = 1e-6) -> np.ndarray:
    """fused_ops.cpp:101-127 on a copy of qkv [T, row]: for each of the first n_q + n_k heads,
    optional norm_row with the q / k weight, then x[i] = t[i] c[i] - t[i+h] s[i],
    x[i+h] = t[i+h] c[i+h] + t[i] s[i+h] (h = D / 2) with cos / sin [T, D]."""
    out = np.array(qkv, F32, copy=True)
    cos = np.asarray(cos, F32).reshape(out.shape[0], D)
    sin = np.asarray(sin, F32).reshape(out.shape[0], D)
    half = D // 2
    for h in range(n_q + n_k):
        x = out[:, h * D:(h + 1) * D]
        w = q_w if h < n_q else k_w
        if w is not None:
            x = rmsnorm(x, w, eps)
        t = x.copy()
        lo = t[:, :half] * cos[:, :half] - t[:, half:] * sin[:, :half]
        hi = t[:, half:] * cos[:, half:] + t[:, :half] * sin[:, half:]
        out[:, h * D:h * D + half] = lo
        out[:, h * D + half:(h + 1) * D] = hi
    return out


def rope_tables(positions: np.ndarray, D: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """cos / sin rows [len(positions), D] of the rotate-half RoPE, built as the reference's
    RotaryEmbedding without scaling (models/layers.py:51-63): inv_freq = 1 / theta^(2i/D) and
    emb = [pos * inv_freq, pos * inv_freq] in float64, cos / sin rounded to float32."""
    inv = 1.0 / theta ** (np.arange(0, D, 2, dtype=np.float64) / D)
    f = np.asarray(positions, np.float64)[:, None] * inv[None, :]
    emb = np.concatenate([f, f], axis=-1)
    return np.cos(emb).astype(F32), np.sin(emb).astype(F32)


# ---- float64 mathematics ------------------------------------------------------------------

def rmsnorm_f64(x, w, eps):
    x = np.asarray(x, np.float64)
    return np.asarray(w, np.float64) * x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)


def silu_mul_f64(gate_up):
    gu = np.asarray(gate_up, np.float64)
    I = gu.shape[-1] // 2
    g, u = gu[..., :I], gu[..., I:]
    return g / (1.0 + np.exp(-g)) * u


def rope_qk_f64(qkv, cos, sin, n_q, n_k, D, q_w=None, k_w=None, eps=1e-6):
    out = np.array(qkv, np.float64, copy=True)
    cos = np.asarray(cos, np.float64).reshape(out.shape[0], D)
    sin = np.asarray(sin, np.float64).reshape(out.shape[0], D)
    half = D // 2
    for h in range(n_q + n_k):
        x = out[:, h * D:(h + 1) * D]
        w = q_w if h < n_q else k_w
        if w is not None:
            x = rmsnorm_f64(x, w, eps)
        rot = np.concatenate([-x[:, half:], x[:, :half]], axis=-1)
        out[:, h * D:(h + 1) * D] = x * cos + rot * sin
    return out
