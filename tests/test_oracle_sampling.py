"""The sampler oracle (oracle/sampling.py) pinned, and the sampler's host (torch) path against it.

Pins of the oracle: the reference's own known answers (tests/test_sampling.py of the
reference: the top-k / top-p / min-p masks of a 5-token row, greedy = argmax, a presence
penalty and a banned token changing the greedy choice), the sampled distribution against the
row's probabilities, and brute force on small rows (top-k keeps exactly the k largest, ties by
index; top-p keeps the shortest prefix of the descending order whose mass reaches top_p,
computed in float64 token by token; min-p keeps p >= min_p * max p).
The torch path of llmserve.sampling (the CPU path of `sample`) must give the oracle's tokens
and in-place logits on the same noise.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sampling as osm

F32 = np.float32


def test_reference_mask_examples():
    lg = np.log(np.array([[0.5, 0.2, 0.15, 0.1, 0.05]], F32))
    m, _ = osm.top_k_top_p_min_p(lg, [2], [1.0], [0.0])
    assert np.isfinite(m).tolist() == [[True, True, False, False, False]]
    m, _ = osm.top_k_top_p_min_p(lg, [-1], [0.8], [0.0])
    assert np.isfinite(m).tolist() == [[True, True, True, False, False]]  # 0.5 + 0.2 < 0.8
    m, _ = osm.top_k_top_p_min_p(lg, [-1], [1.0], [0.3])
    assert np.isfinite(m).tolist() == [[True, True, True, False, False]]  # p >= 0.15


def test_reference_greedy_penalty_banned_examples():
    rng = np.random.default_rng(0)
    lg = rng.standard_normal((3, 50)).astype(F32)
    tok, _, _ = osm.sample(lg, [{"temperature": 0.0}] * 3)
    assert tok.tolist() == lg.argmax(-1).tolist()
    lg = np.zeros((1, 5), F32)
    lg[0, 2] = 1.0
    tok, out, _ = osm.sample(lg, [{"temperature": 0.0, "presence": 2.0, "output": [2]}])
    assert tok.tolist() == [0] and out[0, 2] == -1.0
    tok, _, _ = osm.sample(lg, [{"temperature": 0.0, "banned": [2]}])
    assert tok.tolist() == [0]


def test_distribution_matches_probabilities():
    probs = np.array([0.5, 0.3, 0.15, 0.05], F32)
    n = 20000
    rng = np.random.default_rng(1)
    rows = [{"temperature": 1.0, "noise": rng.exponential(size=4)} for _ in range(n)]
    tok, _, _ = osm.sample(np.log(np.tile(probs, (n, 1))), rows)
    freq = np.bincount(tok, minlength=4) / n
    assert np.allclose(freq, probs, atol=0.015)


@pytest.mark.parametrize("seed", range(20))
def test_masks_brute_force(seed):
    rng = np.random.default_rng(seed)
    V = 12
    x = rng.standard_normal(V).astype(F32)
    x[rng.integers(0, V)] = x[rng.integers(0, V)]  # a tie now and then
    k = int(rng.integers(1, V + 1))
    tp = float(rng.uniform(0.05, 1.0))
    order = sorted(range(V), key=lambda j: (-x[j], j))
    # top-k alone
    m, _ = osm.top_k_top_p_min_p(x[None], [k], [1.0], [0.0])
    assert set(np.flatnonzero(np.isfinite(m[0]))) == set(order[:k])
    # top-p alone: keep while the mass before a token is below top_p (float64, token by token)
    p = np.exp(x.astype(np.float64) - x.max())
    p /= p.sum()
    keep, before = [], 0.0
    for j in order:
        if before < tp:
            keep.append(j)
        before += p[j]
    m, bd = osm.top_k_top_p_min_p(x[None], [-1], [tp], [0.0])
    if not bd[0]:
        assert set(np.flatnonzero(np.isfinite(m[0]))) == set(keep)
    # min-p alone
    mp = float(rng.uniform(0.0, 1.0))
    m, _ = osm.top_k_top_p_min_p(x[None], [-1], [1.0], [mp])
    assert set(np.flatnonzero(np.isfinite(m[0]))) == set(np.flatnonzero(p >= mp * p.max() - 1e-7)) \
        or abs(p / p.max() - mp).min() < 1e-6


def _rows(B, V, seed, dev="cpu"):
    """Mixed rows for the host and device tests: (SampleRows, oracle dicts)."""
    from llmserve.sampling import SampleRow, SamplingParams

    rng = np.random.default_rng(seed)
    srows, orows = [], []
    for i in range(B):
        kind = i % 8
        kw = {}
        if kind == 0:
            kw = dict(temperature=0.0)
        elif kind == 1:
            kw = dict(temperature=0.8, top_k=int(rng.integers(1, 50)))
        elif kind == 2:
            kw = dict(temperature=1.2, top_p=float(rng.uniform(0.3, 0.95)))
        elif kind == 3:
            kw = dict(temperature=0.7, min_p=float(rng.uniform(0.01, 0.2)))
        elif kind == 4:
            kw = dict(temperature=1.0, top_k=int(rng.integers(5, 200)), top_p=0.9, min_p=0.05,
                      presence_penalty=0.5, frequency_penalty=0.3, repetition_penalty=1.3)
        elif kind == 5:
            kw = dict(temperature=0.0, repetition_penalty=1.5, presence_penalty=1.0)
        elif kind == 6:
            kw = dict(temperature=1.0)
        else:
            kw = dict(temperature=0.9, top_p=0.5)
        params = SamplingParams(**kw)
        out = rng.integers(0, V, int(rng.integers(0, 20))).tolist()
        prompt = rng.integers(0, V, int(rng.integers(0, 30))).tolist()
        banned = rng.integers(0, V, 3).tolist() if i % 3 == 0 else []
        allowed = (np.sort(rng.choice(V, min(V, 64), replace=False)) if i % 5 == 4 else None)
        gen_seed = int(rng.integers(0, 2**31))
        gen = torch.Generator().manual_seed(gen_seed)
        srows.append(SampleRow(params, out, prompt, gen, banned,
                               None if allowed is None else torch.from_numpy(allowed)))
        o = {"temperature": params.temperature, "top_k": params.top_k, "top_p": params.top_p,
             "min_p": params.min_p, "presence": params.presence_penalty,
             "frequency": params.frequency_penalty, "repetition": params.repetition_penalty,
             "output": out, "prompt": prompt, "banned": banned,
             "allowed": None if allowed is None else allowed.tolist()}
        if not params.greedy:
            o["noise"] = torch.empty(V).exponential_(
                generator=torch.Generator().manual_seed(gen_seed)).numpy()
        orows.append(o)
    return srows, orows


@pytest.mark.parametrize("B,V,seed", [(16, 1000, 3), (24, 4099, 4)])
def test_host_path_matches_oracle(B, V, seed):
    from llmserve import sampling as sm

    srows, orows = _rows(B, V, seed)
    x = torch.from_numpy(np.random.default_rng(seed + 9).standard_normal((B, V)).astype(F32) * 3)
    want, want_x, border = osm.sample(x.numpy(), orows)
    lg = x.clone()
    got = sm.sample(lg, srows).token_ids
    ok = ~border
    assert np.array_equal(np.asarray(got)[ok], want[ok])
    assert ok.sum() >= B - 2
    assert np.array_equal(lg.numpy(), want_x)  # penalties and masks in place


def test_seeded_rows_independent_of_batch_and_logprobs():
    from llmserve.sampling import SampleRow, SamplingParams, sample

    lg = torch.randn(1, 100, generator=torch.Generator().manual_seed(2))
    a = sample(lg.clone(), [SampleRow(SamplingParams(seed=7, logprobs=3), [], [],
                                      torch.Generator().manual_seed(7))])
    batch = torch.cat([torch.randn(4, 100), lg])
    rows = [SampleRow(SamplingParams(), [], [], None)] * 4 + [
        SampleRow(SamplingParams(seed=7), [], [], torch.Generator().manual_seed(7))]
    b = sample(batch, rows)
    assert a.token_ids[0] == b.token_ids[-1]
    raw = lg.log_softmax(-1)[0]
    assert a.logprobs[0] == pytest.approx(float(raw[a.token_ids[0]]))
    assert [t for t, _ in a.top_logprobs[0]] == raw.topk(3).indices.tolist()


def test_param_validation():
    from llmserve.sampling import SamplingParams

    for bad in (dict(top_p=0), dict(top_k=0), dict(top_k=-2), dict(min_p=1.5), dict(n=0),
                dict(temperature=-1), dict(repetition_penalty=0), dict(max_tokens=0),
                dict(guided_regex="a", guided_choice=["b"])):
        with pytest.raises(ValueError):
            SamplingParams(**bad)
    assert SamplingParams(stop="x").stop == ["x"]
    assert SamplingParams(temperature=0).greedy and not SamplingParams().greedy
