"""The device sampler (llmserve_sample via llmserve.sampling.sample on GPU logits) against the
sampler oracle (oracle/sampling.py) on the same Exp(1) noise, and the reference's own sampler
tests (reference tests/test_sampling.py) run on the GPU.

Bar: identical tokens on every row the oracle does not flag as borderline (its top two p / E
within 1e-5, or a token within rounding of a top-p / min-p cut), at most two flagged rows per
batch; the logits after the call (penalties and masks written in place) equal the oracle's bit
for bit (the same float32 operations, each rounded).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sampling as osm
from test_oracle_sampling import _rows

pytestmark = pytest.mark.gpu
F32 = np.float32


def test_device_path_is_native(gpu):
    from llmserve.sampling import _device_capi

    assert _device_capi(torch.zeros(2, 8, device="cuda")) is not None


@pytest.mark.parametrize("B,V,seed", [(16, 1000, 3), (40, 4099, 4), (64, 151936, 5)])
def test_device_matches_oracle(gpu, B, V, seed):
    from llmserve import sampling as sm

    srows, orows = _rows(B, V, seed)
    x = np.random.default_rng(seed + 9).standard_normal((B, V)).astype(F32) * 3
    want, want_x, border = osm.sample(x, orows)
    lg = torch.from_numpy(x).cuda()
    got = np.asarray(sm.sample(lg, srows).token_ids)
    ok = ~border
    assert ok.sum() >= B - 2
    bad = np.flatnonzero(got[ok] != want[ok])
    assert bad.size == 0, (np.flatnonzero(ok)[bad], got[ok][bad], want[ok][bad])
    assert np.array_equal(lg.cpu().numpy(), want_x)


def test_flat_rows_top_p_and_ties(gpu):
    """Many equal logits (a cut inside a group of ties, resolved by index) and a near-flat
    distribution over the Qwen3 vocabulary (the nucleus holds most of the row)."""
    from llmserve.sampling import SampleRow, SamplingParams, sample

    V = 151936
    x = np.zeros((4, V), F32)
    x[1, ::7] = 1.0  # ties at two levels
    x[2] = np.random.default_rng(1).standard_normal(V).astype(F32) * 0.01
    x[3, :100] = 2.0
    params = [SamplingParams(top_k=50), SamplingParams(top_k=1000, top_p=0.5),
              SamplingParams(top_p=0.9), SamplingParams(top_p=0.3, top_k=70)]
    seeds = [11, 12, 13, 14]
    rows = [SampleRow(p, [], [], torch.Generator().manual_seed(s)) for p, s in zip(params, seeds)]
    orows = [{"temperature": p.temperature, "top_k": p.top_k, "top_p": p.top_p,
              "noise": torch.empty(V).exponential_(generator=torch.Generator().manual_seed(s)).numpy()}
             for p, s in zip(params, seeds)]
    want, _, border = osm.sample(x, orows)
    got = np.asarray(sample(torch.from_numpy(x).cuda(), rows).token_ids)
    assert np.array_equal(got[~border], want[~border]) and (~border).sum() >= 3


def test_reference_examples_on_device(gpu):
    from llmserve.sampling import SampleRow, SamplingParams, sample

    def row(**kw):
        return SampleRow(SamplingParams(**kw), [], [], None)

    logits = torch.randn(3, 50, device="cuda")
    assert sample(logits.clone(), [row(temperature=0)] * 3).token_ids == logits.argmax(-1).tolist()
    logits = torch.zeros(1, 5, device="cuda")
    logits[0, 2] = 1.0
    r = SampleRow(SamplingParams(temperature=0, presence_penalty=2.0), [2], [], None)
    assert sample(logits.clone(), [r]).token_ids == [0]
    r = SampleRow(SamplingParams(temperature=0), [], [], None, banned_token_ids=[2])
    assert sample(logits.clone(), [r]).token_ids == [0]
    # distribution of the exponential race
    probs = torch.tensor([0.5, 0.3, 0.15, 0.05])
    n = 20000
    g = torch.Generator().manual_seed(0)
    toks = torch.tensor(sample(probs.log().expand(n, 4).contiguous().cuda(),
                               [SampleRow(SamplingParams(), [], [], g)] * n).token_ids)
    freq = torch.bincount(toks, minlength=4).float() / n
    assert torch.allclose(freq, probs, atol=0.015)
    # a seeded row samples the same token whatever else is in the batch
    lg = torch.randn(1, 100)
    a = sample(lg.clone().cuda(), [SampleRow(SamplingParams(seed=7), [], [],
                                             torch.Generator().manual_seed(7))])
    batch = torch.cat([torch.randn(4, 100), lg]).cuda()
    rows = [row()] * 4 + [SampleRow(SamplingParams(seed=7), [], [], torch.Generator().manual_seed(7))]
    assert a.token_ids[0] == sample(batch, rows).token_ids[-1]


def test_device_equals_host_path_and_logprobs(gpu):
    """The same rows and noise through the GPU kernel and the CPU torch path; log-probabilities
    come from the raw logits (before penalties)."""
    from llmserve.sampling import sample

    B, V = 24, 3000
    srows, _ = _rows(B, V, 21)
    srows2, _ = _rows(B, V, 21)
    for r in srows + srows2:
        r.params.logprobs = 2
    x = torch.from_numpy(np.random.default_rng(22).standard_normal((B, V)).astype(F32))
    a = sample(x.clone().cuda(), srows)
    b = sample(x.clone(), srows2)
    same = sum(int(p == q) for p, q in zip(a.token_ids, b.token_ids))
    assert same >= B - 2
    raw = x.log_softmax(-1)
    for i, t in enumerate(a.token_ids):
        assert a.logprobs[i] == pytest.approx(float(raw[i, t]), abs=1e-5)
        assert [k for k, _ in a.top_logprobs[i]] == raw[i].topk(2).indices.tolist()
