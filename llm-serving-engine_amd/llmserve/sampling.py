"""Sampling parameters and the batched sampler (drop-in for the reference's llmserve.sampling,
sampling.py:17-204).

``sample(logits, rows)`` takes a [B, V] float32 logits batch and one ``SampleRow`` per row and
returns one token per row, in the reference's order: raw log-probabilities (when asked for),
presence / frequency / repetition penalties and the allowed / banned masks (written into the
logits in place), greedy rows by argmax, the other rows by the exponential race over the
temperature-scaled distribution after top-k / top-p / min-p. For logits on the GPU the work
after the log-probabilities is one launch of ``llmserve_sample`` (csrc/sampling.hip), a
workgroup per row; on the CPU, or without the native library, the same steps run as torch ops.

The Exp(1) noise of a sampled row is drawn as the reference draws it: from the row's
``generator`` (a CPU generator, or torch's default CPU generator when it is None), so a seeded
request samples the same token on either path. A CUDA generator draws the noise on the GPU
instead (no host-to-device copy of V floats per row).
"""

from __future__ import annotations

import ctypes
from collections import Counter
from dataclasses import dataclass, field

import torch

_NEG_INF = float("-inf")
GREEDY_TEMPERATURE = 1e-5  # below this a row is greedy (argmax)


@dataclass
class SamplingParams:
    """Per-request settings (field meanings and checks as the reference's, sampling.py:17-66)."""

    n: int = 1
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = -1  # -1: off
    min_p: float = 0.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    repetition_penalty: float = 1.0
    max_tokens: int = 16
    min_tokens: int = 0
    stop: list[str] = field(default_factory=list)
    stop_token_ids: list[int] = field(default_factory=list)
    ignore_eos: bool = False
    seed: int | None = None
    logprobs: int | None = None  # top log-probabilities per token (0: the sampled one only)
    include_stop_str_in_output: bool = False
    guided_regex: str | None = None
    guided_json: dict | None = None
    guided_choice: list[str] | None = None

    def __post_init__(self) -> None:
        guided = [g for g in (self.guided_regex, self.guided_json, self.guided_choice) if g is not None]
        if len(guided) > 1:
            raise ValueError("use at most one of guided_regex / guided_json / guided_choice")
        if isinstance(self.stop, str):
            self.stop = [self.stop]
        checks = [
            (self.n >= 1, "n must be >= 1"),
            (self.temperature >= 0, "temperature must be >= 0"),
            (0 < self.top_p <= 1, "top_p must be in (0, 1]"),
            (self.top_k == -1 or self.top_k >= 1, "top_k must be -1 (disabled) or >= 1"),
            (0 <= self.min_p <= 1, "min_p must be in [0, 1]"),
            (self.repetition_penalty > 0, "repetition_penalty must be > 0"),
            (self.max_tokens >= 1, "max_tokens must be >= 1"),
        ]
        for ok, msg in checks:
            if not ok:
                raise ValueError(msg)

    @property
    def guided_pattern(self) -> str | None:
        """The regular expression the completion must match. JSON schemas and choice lists are
        compiled to one by the reference's structured-output package, which this package does
        not carry (only the sampler's allowed-token mask is here)."""
        if self.guided_regex is not None:
            return self.guided_regex
        if self.guided_json is not None or self.guided_choice is not None:
            raise NotImplementedError("guided_json / guided_choice need the structured-output "
                                      "compiler, which is outside this package")
        return None

    @property
    def greedy(self) -> bool:
        return self.temperature < GREEDY_TEMPERATURE


@dataclass
class SampleRow:
    """What the sampler needs of one row of the logits batch."""

    params: SamplingParams
    output_token_ids: list[int]
    prompt_token_ids: list[int]
    generator: torch.Generator | None
    banned_token_ids: list[int] = field(default_factory=list)  # e.g. EOS before min_tokens
    allowed_token_ids: torch.Tensor | None = None  # structured output: only these tokens


@dataclass
class SamplerOutput:
    token_ids: list[int]
    logprobs: list[float] | None  # log-probability of the sampled token (raw distribution)
    top_logprobs: list[list[tuple[int, float]]] | None


def _penalized(p: SamplingParams) -> bool:
    return p.presence_penalty != 0 or p.frequency_penalty != 0 or p.repetition_penalty != 1.0


def apply_penalties(logits: torch.Tensor, rows: list[SampleRow]) -> torch.Tensor:
    """OpenAI presence / frequency penalties over the generated tokens, then the HF repetition
    penalty over prompt + generated tokens (x / r above 0, x * r otherwise), in place."""
    V = logits.shape[1]
    for i, r in enumerate(rows):
        p = r.params
        if not _penalized(p):
            continue
        if r.output_token_ids and (p.presence_penalty != 0 or p.frequency_penalty != 0):
            cnt = torch.bincount(torch.as_tensor(r.output_token_ids, dtype=torch.long), minlength=V)
            cnt = cnt.to(device=logits.device, dtype=logits.dtype)
            logits[i] -= p.frequency_penalty * cnt + p.presence_penalty * (cnt > 0).to(logits.dtype)
        if p.repetition_penalty != 1.0:
            seen = sorted(set(r.prompt_token_ids).union(r.output_token_ids))
            if seen:
                ix = torch.as_tensor(seen, dtype=torch.long, device=logits.device)
                v = logits[i, ix]
                logits[i, ix] = torch.where(v > 0, v / p.repetition_penalty, v * p.repetition_penalty)
    return logits


def _top_k_top_p_min_p(logits: torch.Tensor, top_k: torch.Tensor, top_p: torch.Tensor,
                       min_p: torch.Tensor) -> torch.Tensor:
    """-inf outside each row's top-k / nucleus / min-p set: ranks >= k, tokens whose preceding
    mass under the row's softmax reaches top_p (the first token always stays), then tokens
    below min_p times the largest remaining probability."""
    V = logits.shape[1]
    if bool((top_k > 0).any()) or bool((top_p < 1).any()):
        vals, order = logits.sort(dim=-1, descending=True)
        k = torch.where(top_k > 0, top_k, torch.full_like(top_k, V)).to(logits.device)
        rank = torch.arange(V, device=logits.device).expand_as(vals)
        prob = vals.softmax(-1)
        before = prob.cumsum(-1) - prob
        drop = (rank >= k[:, None]) | (before >= top_p.to(logits.device)[:, None])
        logits = torch.empty_like(logits).scatter_(1, order, vals.masked_fill(drop, _NEG_INF))
    if bool((min_p > 0).any()):
        prob = logits.softmax(-1)
        floor = prob.amax(-1, keepdim=True) * min_p.to(logits.device)[:, None]
        logits = logits.masked_fill(prob < floor, _NEG_INF)
    return logits


def _exponential(shape: tuple[int, ...], gen: torch.Generator | None) -> torch.Tensor:
    """Exp(1) noise from `gen` (CPU, or torch's default CPU generator) or on gen's GPU."""
    if gen is not None and gen.device.type != "cpu":
        return torch.empty(shape, device=gen.device).exponential_(generator=gen)
    return torch.empty(shape).exponential_(generator=gen)


def _mask_rows(logits: torch.Tensor, rows: list[SampleRow]) -> None:
    for i, r in enumerate(rows):
        if r.allowed_token_ids is not None:
            ix = torch.as_tensor(r.allowed_token_ids, device=logits.device)
            keep = logits[i, ix]
            logits[i] = _NEG_INF
            logits[i, ix] = keep
        if r.banned_token_ids:
            logits[i, torch.as_tensor(r.banned_token_ids, device=logits.device)] = _NEG_INF


def _sample_torch(logits: torch.Tensor, rows: list[SampleRow]) -> torch.Tensor:
    """Penalties, masks and the token choice as torch ops (the CPU path)."""
    B = logits.shape[0]
    apply_penalties(logits, rows)
    _mask_rows(logits, rows)
    greedy = [i for i, r in enumerate(rows) if r.params.greedy]
    if len(greedy) == B:
        return logits.argmax(-1)
    tokens = torch.empty(B, dtype=torch.long, device=logits.device)
    if greedy:
        gi = torch.as_tensor(greedy, device=logits.device)
        tokens[gi] = logits.index_select(0, gi).argmax(-1)
    todo = [i for i in range(B) if not rows[i].params.greedy]
    ti = torch.as_tensor(todo, device=logits.device)
    temps = torch.tensor([rows[i].params.temperature for i in todo], device=logits.device)
    sub = _top_k_top_p_min_p(
        logits.index_select(0, ti) / temps[:, None],
        torch.tensor([rows[i].params.top_k for i in todo]),
        torch.tensor([rows[i].params.top_p for i in todo]),
        torch.tensor([rows[i].params.min_p for i in todo]))
    noise = torch.stack([_exponential((logits.shape[1],), rows[i].generator).to(logits.device)
                         for i in todo])
    tokens[ti] = (sub.softmax(-1) / noise).argmax(-1)
    return tokens


def _csr(lists: list[list[int]], dev) -> tuple[torch.Tensor, torch.Tensor]:
    ptr = [0]
    for x in lists:
        ptr.append(ptr[-1] + len(x))
    flat = [t for x in lists for t in x] or [0]
    return (torch.tensor(ptr, dtype=torch.long).to(dev, non_blocking=True),
            torch.tensor(flat, dtype=torch.long).to(dev, non_blocking=True))


def _sample_device(logits: torch.Tensor, rows: list[SampleRow], capi) -> torch.Tensor:
    """One llmserve_sample launch over the batch (penalties and masks written in place)."""
    from ._native import check

    B, V = logits.shape
    dev = logits.device
    params = [r.params for r in rows]
    outs, cnts, seen, allow, has_allow, ban = [], [], [], [], [], []
    for r, p in zip(rows, params):
        if r.output_token_ids and (p.presence_penalty != 0 or p.frequency_penalty != 0):
            c = Counter(r.output_token_ids)
            outs.append(list(c.keys()))
            cnts.append(list(c.values()))
        else:
            outs.append([])
            cnts.append([])
        seen.append(sorted(set(r.prompt_token_ids).union(r.output_token_ids))
                    if p.repetition_penalty != 1.0 else [])
        has_allow.append(r.allowed_token_ids is not None)
        allow.append([] if r.allowed_token_ids is None else
                     torch.as_tensor(r.allowed_token_ids).reshape(-1).tolist())
        ban.append(list(r.banned_token_ids))
    out_ptr, out_ids = _csr(outs, dev)
    out_cnt = torch.tensor([c for x in cnts for c in x] or [0], dtype=torch.int32).to(dev)
    seen_ptr, seen_ids = _csr(seen, dev)
    allow_ptr, allow_ids = _csr(allow, dev)
    ban_ptr, ban_ids = _csr(ban, dev)
    f32 = torch.tensor([[0.0 if p.greedy else p.temperature for p in params],
                        [p.top_p for p in params], [p.min_p for p in params],
                        [p.presence_penalty for p in params],
                        [p.frequency_penalty for p in params],
                        [p.repetition_penalty for p in params]], dtype=torch.float32).to(dev)
    top_k = torch.tensor([p.top_k for p in params], dtype=torch.int32).to(dev)
    flags = torch.tensor(has_allow, dtype=torch.uint8).to(dev)
    todo = [i for i, p in enumerate(params) if not p.greedy]
    slot = {i: n for n, i in enumerate(todo)}
    noise_row = torch.tensor([slot.get(i, 0) for i in range(B)], dtype=torch.long).to(dev)
    if todo:
        noise = torch.stack([_exponential((V,), rows[i].generator).to(dev) for i in todo])
    else:
        noise = torch.ones(1, V, device=dev)
    use_topkp = any(params[i].top_k > 0 or params[i].top_p < 1 for i in todo)
    use_minp = any(params[i].min_p > 0 for i in todo)
    tokens = torch.empty(B, dtype=torch.long, device=dev)

    def p(t):
        return ctypes.c_void_p(t.data_ptr())

    check(capi.llmserve_sample(
        p(logits), B, V, p(f32[0]), p(top_k), p(f32[1]), p(f32[2]), p(f32[3]), p(f32[4]),
        p(f32[5]), p(out_ptr), p(out_ids), p(out_cnt), p(seen_ptr), p(seen_ids), p(allow_ptr),
        p(allow_ids), p(flags), p(ban_ptr), p(ban_ids), p(noise), p(noise_row), int(use_topkp),
        int(use_minp), p(tokens), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
    return tokens


def _device_capi(logits: torch.Tensor):
    """The C ABI when the batch can run on the GPU kernel (None: the torch path)."""
    if not logits.is_cuda or logits.dtype != torch.float32 or logits.dim() != 2:
        return None
    from .kernels import native_available

    if not native_available():
        return None
    from ._native import capi

    return capi()


def sample(logits: torch.Tensor, rows: list[SampleRow]) -> SamplerOutput:
    """logits: [B, V] float32 (penalties and masks are written into it, as the reference does;
    a non-contiguous tensor is worked on as a contiguous copy). One token per row."""
    want = any(r.params.logprobs is not None for r in rows)
    raw = logits.log_softmax(-1) if want else None
    logits = logits.contiguous() if not logits.is_contiguous() else logits
    capi = _device_capi(logits)
    tokens = _sample_device(logits, rows, capi) if capi is not None else _sample_torch(logits, rows)
    token_list = tokens.tolist()
    if not want:
        return SamplerOutput(token_list, None, None)
    lps, tops = [], []
    for i, r in enumerate(rows):
        lps.append(float(raw[i, token_list[i]]))
        k = r.params.logprobs or 0
        if k > 0:
            v, ix = raw[i].topk(k)
            tops.append(list(zip(ix.tolist(), v.tolist(), strict=True)))
        else:
            tops.append([])
    return SamplerOutput(token_list, lps, tops)


__all__ = ["GREEDY_TEMPERATURE", "SampleRow", "SamplerOutput", "SamplingParams",
           "apply_penalties", "sample"]
