"""ORACLE (test infrastructure only) — float64 references of the path's mathematics.

These fix what the kernels must compute independently of any summation order:
  * weight-only linears: y = x @ W_deq^T with W_deq the float32 dequantized weight;
  * paged decode: softmax(scale * q . k_deq) @ v_deq over each sequence's context, slots
    from the block table.
Pinned by tests/test_oracle_math.py with brute-force loops on tiny inputs, torch SDPA and
closed forms (uniform attention, one-token contexts).
"""

from __future__ import annotations

import numpy as np

from oracle import quant as oq


def linear_f64(x: np.ndarray, w_deq: np.ndarray) -> np.ndarray:
    """y[m, n] = sum_k x[m, k] w[n, k] in float64."""
    return np.asarray(x, np.float64) @ np.asarray(w_deq, np.float64).T


def int8_linear_f64(x, q, scale):
    return linear_f64(x, oq.int8_dequantize(q, scale))


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32: the rounding of
    torch's float32 -> bfloat16 cast and of gfx950's v_cvt_pk_bf16_f32. Finite inputs only.
    Pinned by tests/test_oracle_math.py against torch's CPU cast on random values, exact
    ties (both parities), signed zeros, subnormals and values that round up to a new binade."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return r.astype(np.uint32).view(np.float32)


def int8_linear_prefill_f64(x, q, scale, round_x: bool = True):
    """Int8Linear's large-M path (reference quant.py:71-72): x @ (q * scale[:, None]).T in
    float64. With round_x, x is first rounded to bfloat16 — what the bf16 matrix-core GEMM
    computes exactly up to its float32 accumulation; without, the weight-only product the
    stated bf16 tolerance is measured against."""
    x = np.asarray(x, np.float32)
    xr = bf16_round(x) if round_x else x
    y = np.asarray(xr, np.float64) @ np.asarray(q, np.float64).T
    return y * np.asarray(scale, np.float64)[None, :]


def int4_linear_f64(x, nib, g_scale, g_zero, group_size, inv_act_scale=None):
    """Int4Linear.forward: x * inv_act_scale (float32), then x @ dequantize()^T."""
    x = np.asarray(x, np.float32)
    if inv_act_scale is not None:
        x = (x * inv_act_scale[None, :]).astype(np.float32)
    return linear_f64(x, oq.int4_dequantize(nib, g_scale, g_zero, group_size))


def context_slots(table: np.ndarray, ctx: int, block_size: int) -> np.ndarray:
    t = np.arange(ctx)
    return table[t // block_size].astype(np.int64) * block_size + t % block_size


def paged_decode_f64(q, k_deq, v_deq, block_tables, context_lens, block_size, scale):
    """out[b, hq] = softmax_t(scale * q[b, hq] . k[slot_t, hq // G]) @ v[slot_t, hq // G].

    q [B, Hq, D]; k_deq / v_deq [num_slots, Hk, D] (dequantized caches); returns float64.
    """
    q = np.asarray(q, np.float64)
    B, Hq, D = q.shape
    Hk = k_deq.shape[1]
    G = Hq // Hk
    out = np.zeros((B, Hq, D))
    for b in range(B):
        ctx = int(context_lens[b])
        slots = context_slots(np.asarray(block_tables[b]), ctx, block_size)
        kb = np.asarray(k_deq[slots], np.float64)  # [ctx, Hk, D]
        vb = np.asarray(v_deq[slots], np.float64)
        for hq in range(Hq):
            h = hq // G
            s = scale * (kb[:, h, :] @ q[b, hq])
            s = s - s.max()
            p = np.exp(s)
            out[b, hq] = (p @ vb[:, h, :]) / p.sum()
    return out


def kv_dequantize(data: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """QuantizedKV.rows (reference attention.py:164-166): data * scale[..., None] in float32."""
    return (data.astype(np.float32) * scale[..., None]).astype(np.float32)


def paged_rows_f64(q, k_deq, v_deq, block_tables, row_table, row_context, block_size, scale):
    """Query row r attends, with paged_decode_f64, to the first row_context[r] tokens of
    block-table row row_table[r] (a prefill token at position p has row_context p + 1: the
    causal mask of the reference's prefill SDPA, attention.py:114-124)."""
    tables = np.asarray(block_tables)[np.asarray(row_table, np.int64)]
    return paged_decode_f64(q, k_deq, v_deq, tables, row_context, block_size, scale)


def step_rows(q_lens, ctx_lens, block_tables, block_size):
    """(slot_mapping, row_table, row_context) of a ragged batch, built the way the reference's
    AttentionMetadata.build walks it (attention.py:68-84): per sequence the context slots
    blocks[:, None] * bs + arange(bs), flattened and cut at ctx, of which the last q_len are
    the new tokens' slots. Plain Python loops (small inputs)."""
    slots_out, rows, ctx_out = [], [], []
    for s, (q_len, ctx, table) in enumerate(zip(q_lens, ctx_lens, block_tables)):
        n = -(-ctx // block_size)
        ctx_slots = [b * block_size + o for b in table[:n] for o in range(block_size)][:ctx]
        for j in range(q_len):
            p = ctx - q_len + j
            slots_out.append(ctx_slots[p])
            rows.append(s)
            ctx_out.append(p + 1)
    return (np.array(slots_out, np.int64), np.array(rows, np.int64), np.array(ctx_out, np.int64))
