"""ORACLE (test infrastructure only) — one greedy decode step of a quantized Qwen3-style model,
as the reference runs it: CausalLM._forward_fused (models/transformer.py:144-190), then
compute_logits (:192-193) and the greedy fast path of the sampler (sampling.py:169-170).

``decode_step`` composes this directory's pinned parts in the reference's order, float32:
  * embedding row, fused_ops.rmsnorm with layer 0's input norm (transformer.py:151-155);
  * per layer: Int4Linear qkv (cpu.int4_linear, the reference's int8_gemv.cpp kernel),
    fused_ops.rope_qk with the Qwen3 q/k norms (:157-171), then paged_attention
    (attention.py:231-273): q * q_mult and k / smooth, quantize and write this token's K and V
    (quant.kv_quantize, QuantizedKV.write), cpu.paged_decode_int8 over the int8 cache;
    o_proj, add_rmsnorm with the post-attention norm (:184), gate_up, silu_mul, down, and
    add_rmsnorm with the next layer's input norm or the final norm (:185-189);
  * lm_head (fp32 matrix or Int4Linear) and the first index of the row maximum (torch.argmax).
The batch is decode-only: token b sits at position ctx[b] - 1 and its KV goes to the slot
block_tables[b, pos // block_size] * block_size + pos % block_size.

``decode_step_plain_f64`` is the same model written the plain way (HF-style: explicit residual
adds, norms recomputed, RoPE as q * cos + rotate_half(q) * sin from angles computed in float64,
attention by math_ref.paged_decode_f64) in float64. tests/test_oracle_step.py pins
``decode_step`` against it at the reference's fused-vs-plain tolerance (1e-4,
tests/test_fused_ops.py:31-40) and checks the KV rows each writes.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from oracle import cpu as oc
from oracle import fused_ops as ofo
from oracle import math_ref as mr
from oracle import quant as oq

F32 = np.float32


@dataclass
class Int4W:
    """Int4Linear buffers (reference quant.py:94-121)."""

    nib: np.ndarray  # uint8 [N, K/2]
    g_scale: np.ndarray  # [N, G]
    g_zero: np.ndarray  # [N, G]
    inv: np.ndarray | None  # inv_act_scale [K]
    group: int


@dataclass
class Layer:
    input_layernorm: np.ndarray
    post_attention_layernorm: np.ndarray
    q_norm: np.ndarray | None
    k_norm: np.ndarray | None
    qkv: Int4W
    o: Int4W
    gate_up: Int4W
    down: Int4W


@dataclass
class Weights:
    embed: np.ndarray  # [V, H]
    norm: np.ndarray  # final norm [H]
    lm_head: np.ndarray | Int4W  # fp32 [V, H] or Int4W
    layers: list[Layer] = field(default_factory=list)


@dataclass
class LayerCache:
    """QuantizedKV pair of one layer: int8 data [S, Hk, D] and fp32 scales [S, Hk]."""

    kd: np.ndarray
    ks: np.ndarray
    vd: np.ndarray
    vs: np.ndarray
    smooth: np.ndarray | None = None  # [Hk, D]

    def copy(self) -> LayerCache:
        return LayerCache(self.kd.copy(), self.ks.copy(), self.vd.copy(), self.vs.copy(),
                          None if self.smooth is None else self.smooth.copy())


def _lin(x, w: Int4W):
    return oc.int4_linear(x, w.nib, w.g_scale, w.g_zero, w.group, w.inv)


def _lin64(x, w: Int4W):
    return mr.int4_linear_f64(np.asarray(x, F32), w.nib, w.g_scale, w.g_zero, w.group, w.inv)


def token_slots(block_tables: np.ndarray, ctx: np.ndarray, block_size: int) -> np.ndarray:
    pos = np.asarray(ctx, np.int64) - 1
    b = np.arange(len(pos))
    return block_tables[b, pos // block_size].astype(np.int64) * block_size + pos % block_size


def q_mult(smooth: np.ndarray, n_q: int) -> np.ndarray:
    """QuantizedKV._q_mult: the smoothing vector repeated per GQA group (attention.py:150)."""
    return np.repeat(np.asarray(smooth, F32), n_q // smooth.shape[0], axis=0)


def decode_step(W: Weights, cfg, ids, ctx, block_tables, caches: list[LayerCache],
                block_size: int, cos_tab: np.ndarray, sin_tab: np.ndarray, write_kv: bool = True):
    """float32, the reference's fused order. ``caches`` are updated in place with this step's
    K/V (with ``write_kv=False`` they must already hold them: attention then reads the rows
    another implementation wrote, so that a one-step rounding difference of a quantized K/V
    value does not enter the comparison of the logits). Returns (logits [B, V] float32,
    next ids [B], per layer (k data, k scale, v data, v scale) of this step's rows)."""
    nq, nk, D, eps = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.rms_norm_eps
    ids, ctx = np.asarray(ids, np.int64), np.asarray(ctx, np.int64)
    B = len(ids)
    pos = ctx - 1
    slots = token_slots(block_tables, ctx, block_size)
    cos, sin = cos_tab[pos], sin_tab[pos]
    scale = float(D) ** -0.5
    x = W.embed[ids].astype(F32)
    h = ofo.rmsnorm(x, W.layers[0].input_layernorm, eps)
    n = len(W.layers)
    rows = []
    for i, L in enumerate(W.layers):
        c = caches[i]
        qkv = ofo.rope_qk(_lin(h, L.qkv), cos, sin, nq, nk, D, L.q_norm, L.k_norm, eps)
        q = qkv[:, :nq * D].reshape(B, nq, D)
        k = qkv[:, nq * D:(nq + nk) * D].reshape(B, nk, D)
        v = qkv[:, (nq + nk) * D:].reshape(B, nk, D)
        qm = None
        if c.smooth is not None:
            k = oq.kv_smooth(k, c.smooth)
            qm = q_mult(c.smooth, nq)
        kq, ks = oq.kv_quantize(k)
        vq, vs = oq.kv_quantize(v)
        rows.append((kq, ks, vq, vs))
        if write_kv:
            c.kd[slots], c.ks[slots], c.vd[slots], c.vs[slots] = kq, ks, vq, vs
        o = oc.paged_decode_int8(q, c.kd, c.vd, c.ks, c.vs, block_tables, ctx, block_size, scale,
                                 0, qm)
        attn = _lin(o.reshape(B, nq * D), L.o)
        x, h = ofo.add_rmsnorm(x, attn, L.post_attention_layernorm, eps)
        down = _lin(ofo.silu_mul(_lin(h, L.gate_up)), L.down)
        nxt = W.layers[i + 1].input_layernorm if i + 1 < n else W.norm
        x, h = ofo.add_rmsnorm(x, down, nxt, eps)
    if isinstance(W.lm_head, Int4W):
        logits = _lin(h, W.lm_head)
    else:
        logits = (h @ np.asarray(W.lm_head, F32).T).astype(F32)
    return logits, argmax_first(logits), rows


def argmax_first(logits: np.ndarray) -> np.ndarray:
    """torch.argmax over the last axis: first index of the maximum, NaN above every number."""
    lg = np.asarray(logits)
    out = np.argmax(lg, axis=-1)  # numpy also returns the first NaN, else the first maximum
    return out.astype(np.int64)


# ---- plain float64 restatement ------------------------------------------------------------

def _rms64(x, w, eps):
    x = np.asarray(x, np.float64)
    return np.asarray(w, np.float64) * x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)


def _rope64(t, pos, theta):
    """t [B, H, D]: t * cos + rotate_half(t) * sin, angles pos * theta^(-2i/D) in float64."""
    D = t.shape[-1]
    ang = np.asarray(pos, np.float64)[:, None] * theta ** (-np.arange(0, D, 2) / D)[None, :]
    ang = np.concatenate([ang, ang], -1)[:, None, :]
    rot = np.concatenate([-t[..., D // 2:], t[..., :D // 2]], -1)
    return t * np.cos(ang) + rot * np.sin(ang)


def decode_step_plain_f64(W: Weights, cfg, ids, ctx, block_tables, caches: list[LayerCache],
                          block_size: int, write_kv: bool = True):
    """float64 plain forward of the same step; ``caches`` are updated in place (the new K/V
    rows quantized by the float32 quantizer, the cache format; with ``write_kv=False`` they
    must already hold this step's rows, as in ``decode_step``). Returns logits float64."""
    nq, nk, D, eps = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.rms_norm_eps
    ids, ctx = np.asarray(ids, np.int64), np.asarray(ctx, np.int64)
    B = len(ids)
    pos = ctx - 1
    slots = token_slots(block_tables, ctx, block_size)
    x = np.asarray(W.embed, np.float64)[ids]
    for i, L in enumerate(W.layers):
        c = caches[i]
        h = _rms64(x, L.input_layernorm, eps)
        qkv = _lin64(h, L.qkv)
        q = qkv[:, :nq * D].reshape(B, nq, D)
        k = qkv[:, nq * D:(nq + nk) * D].reshape(B, nk, D)
        v = qkv[:, (nq + nk) * D:].reshape(B, nk, D)
        if L.q_norm is not None:
            q, k = _rms64(q, L.q_norm, eps), _rms64(k, L.k_norm, eps)
        q, k = _rope64(q, pos, cfg.rope_theta), _rope64(k, pos, cfg.rope_theta)
        if c.smooth is not None:
            k = k / np.asarray(c.smooth, np.float64)
            q = q * np.repeat(np.asarray(c.smooth, np.float64), nq // nk, axis=0)
        if write_kv:
            c.kd[slots], c.ks[slots] = oq.kv_quantize(k.astype(F32))
            c.vd[slots], c.vs[slots] = oq.kv_quantize(v.astype(F32))
        o = mr.paged_decode_f64(q, mr.kv_dequantize(c.kd, c.ks), mr.kv_dequantize(c.vd, c.vs),
                                block_tables, ctx, block_size, float(D) ** -0.5)
        x = x + _lin64(o.reshape(B, nq * D), L.o)
        h = _rms64(x, L.post_attention_layernorm, eps)
        gu = _lin64(h, L.gate_up)
        inter = gu.shape[1] // 2
        g, u = gu[:, :inter], gu[:, inter:]
        x = x + _lin64(g / (1.0 + np.exp(-g)) * u, L.down)
    h = _rms64(x, W.norm, eps)
    if isinstance(W.lm_head, Int4W):
        return _lin64(h, W.lm_head)
    return h @ np.asarray(W.lm_head, np.float64).T


# ---- random models and caches for tests -----------------------------------------------------

def random_model(cfg, group: int, seed: int, lm_int4: bool = False, awq: bool = True) -> Weights:
    """Seeded random weights quantized by the oracle's quantizers: linears N(0, 0.02) with AWQ
    scales from synthetic |activation| means (1% of channels x 20), norms 1 + N(0, 0.1), the
    LM head tied to the embedding (quantized too with ``lm_int4``, as quantize_lm_head)."""
    rng = np.random.default_rng(seed)
    H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    nq, nk, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim

    def lin(n_out, n_in, w=None):
        if w is None:
            w = (rng.standard_normal((n_out, n_in)) * 0.02).astype(F32)
        s = None
        if awq:
            a = np.abs(rng.standard_normal(n_in)).astype(F32) + F32(0.5)
            a[rng.choice(n_in, max(1, n_in // 100), replace=False)] *= 20
            s = np.sqrt(a).astype(F32)
        return Int4W(*oq.int4_quantize_pack(w, group, s), group)

    def norm(n):
        return (1 + 0.1 * rng.standard_normal(n)).astype(F32)

    layers = [Layer(norm(H), norm(H), norm(D) if cfg.qk_norm else None,
                    norm(D) if cfg.qk_norm else None, lin((nq + 2 * nk) * D, H), lin(H, nq * D),
                    lin(2 * I, H), lin(H, I)) for _ in range(cfg.num_hidden_layers)]
    embed = (rng.standard_normal((V, H)) * 0.02).astype(F32)
    lm = lin(V, H, embed) if lm_int4 else embed  # tied embeddings (Qwen3-0.6B)
    return Weights(embed, norm(H), lm, layers)


def random_caches(cfg, num_slots: int, seed: int, smooth: bool = True) -> list[LayerCache]:
    """int8 caches of random content (as after a prefill): data uniform in [-127, 127],
    scales in [0.005, 0.03], smoothing vectors with mean 1 per head."""
    rng = np.random.default_rng(seed)
    nk, D = cfg.num_key_value_heads, cfg.head_dim
    out = []
    for _ in range(cfg.num_hidden_layers):
        def data():
            return rng.integers(-127, 128, (num_slots, nk, D)).astype(np.int8)

        def sc():
            return rng.uniform(0.005, 0.03, (num_slots, nk)).astype(F32)

        s = None
        if smooth:
            s = rng.uniform(0.5, 2.0, (nk, D)).astype(F32)
            s = (s / s.mean(-1, keepdims=True)).astype(F32)
        out.append(LayerCache(data(), sc(), data(), sc(), s))
    return out
