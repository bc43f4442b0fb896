"""ORACLE (test infrastructure only) — the reference's batched sampler in numpy, float32.

Restates sampling.sample (reference sampling.py:151-189) with its helpers apply_penalties
(:100-120) and _top_k_top_p_min_p (:123-143) for rows given as plain dicts, with the Exp(1)
noise of each sampled row passed in (the reference draws it from the row's generator,
:146-148, 183-186), so the HIP sampler and this restatement can be run on the same noise.

Ties in the descending sort of the top-k / top-p step are broken by ascending index (a stable
sort), the order the HIP kernel uses. Softmax is computed in float64 and rounded once to
float32 (torch's CPU softmax is within an ulp of that), the cumulative sum accumulates in
float64 as torch's CPU cumsum does. Also returns, per row, whether the choice is borderline:
the top two values of p / E within 1e-5 (relative) of each other, a token whose preceding mass
lies within 1e-5 of top_p, or a probability within 1e-6 of the min-p floor (where an ulp of
rounding decides which side of a cut a token falls).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def _softmax(x: np.ndarray) -> np.ndarray:
    """softmax of float32 values, computed in float64 and rounded once to float32."""
    x = np.asarray(x, np.float64)
    m = x.max(-1, keepdims=True)
    e = np.exp(x - m)
    return (e / e.sum(-1, keepdims=True)).astype(F32)


def apply_penalties(logits: np.ndarray, rows: list[dict]) -> None:
    """In place, as sampling.py:100-120: x - (f * count + p * (count > 0)) over the generated
    tokens, then the repetition penalty (x / r above 0, x * r otherwise) over prompt +
    generated tokens."""
    V = logits.shape[1]
    for i, r in enumerate(rows):
        pres, freq, rep = (F32(r.get("presence", 0.0)), F32(r.get("frequency", 0.0)),
                           F32(r.get("repetition", 1.0)))
        out, prompt = r.get("output", []), r.get("prompt", [])
        if pres == 0 and freq == 0 and rep == 1:
            continue
        if out and (pres != 0 or freq != 0):
            cnt = np.bincount(np.asarray(out, np.int64), minlength=V).astype(F32)
            logits[i] = logits[i] - (freq * cnt + pres * (cnt > 0).astype(F32))
        if rep != 1:
            seen = np.asarray(sorted(set(prompt) | set(out)), np.int64)
            if seen.size:
                v = logits[i, seen]
                logits[i, seen] = np.where(v > 0, v / rep, v * rep).astype(F32)


def top_k_top_p_min_p(logits: np.ndarray, top_k, top_p, min_p):
    """(masked logits, borderline rows) as sampling.py:123-143, stable descending sort."""
    x = np.asarray(logits, F32).copy()
    B, V = x.shape
    top_k, top_p, min_p = (np.asarray(top_k), np.asarray(top_p, F32), np.asarray(min_p, F32))
    border = np.zeros(B, bool)
    if (top_k > 0).any() or (top_p < 1).any():
        order = np.argsort(-x, axis=-1, kind="stable")
        vals = np.take_along_axis(x, order, -1)
        k = np.where(top_k > 0, top_k, V)
        rank = np.arange(V)[None, :]
        prob = _softmax(vals)
        # torch's CPU cumsum of float32 accumulates in float64 and rounds each output
        before = (np.cumsum(prob, -1, dtype=np.float64).astype(F32) - prob).astype(F32)
        drop = (rank >= k[:, None]) | (before >= top_p[:, None])
        near = np.abs(before.astype(np.float64) - top_p[:, None]) < 1e-5
        border |= (near & (top_p[:, None] < 1) & (rank < k[:, None])).any(-1)
        vals = np.where(drop, F32(-np.inf), vals)
        out = np.empty_like(x)
        np.put_along_axis(out, order, vals, -1)
        x = out
    if (min_p > 0).any():
        prob = _softmax(x)
        floor = (prob.max(-1, keepdims=True) * min_p[:, None]).astype(F32)
        near = np.abs(prob.astype(np.float64) - floor) <= 1e-6 * floor
        border |= (near & np.isfinite(x) & (min_p[:, None] > 0)).any(-1)
        x = np.where(prob < floor, F32(-np.inf), x).astype(F32)
    return x, border


def sample(logits: np.ndarray, rows: list[dict]):
    """(tokens [B], logits after penalties and masks, borderline [B]). A row dict holds
    temperature, top_k, top_p, min_p, presence, frequency, repetition, output, prompt, banned,
    allowed (None: no mask) and, for a sampled row, noise [V]."""
    x = np.asarray(logits, F32).copy()
    B, V = x.shape
    apply_penalties(x, rows)
    for i, r in enumerate(rows):
        if r.get("allowed") is not None:
            keep = x[i, r["allowed"]]
            x[i] = -np.inf
            x[i, r["allowed"]] = keep
        if r.get("banned"):
            x[i, r["banned"]] = -np.inf
    tokens = np.zeros(B, np.int64)
    border = np.zeros(B, bool)
    greedy = [i for i, r in enumerate(rows) if r.get("temperature", 1.0) < 1e-5]
    for i in greedy:
        tokens[i] = int(np.argmax(x[i]))
    todo = [i for i in range(B) if i not in greedy]
    if todo:
        temps = np.asarray([rows[i].get("temperature", 1.0) for i in todo], F32)
        sub = (x[todo] / temps[:, None]).astype(F32)
        sub, bd = top_k_top_p_min_p(sub, [rows[i].get("top_k", -1) for i in todo],
                                    [rows[i].get("top_p", 1.0) for i in todo],
                                    [rows[i].get("min_p", 0.0) for i in todo])
        q = _softmax(sub) / np.stack([np.asarray(rows[i]["noise"], F32) for i in todo])
        for n, i in enumerate(todo):
            tokens[i] = int(np.argmax(q[n]))
            top2 = np.sort(q[n])[-2:]
            border[i] = bd[n] or (top2[0] > 0 and (top2[1] - top2[0]) <= 1e-5 * top2[1])
    return tokens, x, border


__all__ = ["apply_penalties", "sample", "top_k_top_p_min_p"]
