"""CPU simulation of the decode chain's hand-off schedule (llm-serving-engine_amd/csrc/
decode_chain.hip), run before the kernel ever runs on a GPU.

The kernel's workgroups are restated as Python generators that perform the same sequence of
hand-off operations with the same index formulas. First this layer's attention (MLP mode):
the range length Q and ranges per row R come from the longest context (attn_plan), workgroup
w < M R puts the partials of range w % R of row w / R (its kv heads' query heads, ranges with
tokens only) into exa; workgroup grid - 1 - i (i < M n_q) takes the partials of the
ceil(ctx / Q) ranges of row i / n_q, head i % n_q, and puts the merged row into exb. Then
MLP group w takes all of exb, puts o_proj rows 8w..8w+7 into ex1, takes all of ex1, puts
silu * up channels [C w, C (w + 1)) into ex2, takes all of ex2, puts
down rows 8w..8w+7 into ex3 and (last layer) takes all of ex3; a head group takes all of ex1,
then all of ex3; every group then counts itself finished and the last one advances the tag
base. A word is (tag, value); a take completes only when every word it needs carries the
launch's tag.

Checked, under many random interleavings (including workgroups that start late, and several
launches in a row on one workspace): no schedule deadlocks while all groups are resident; every
value a consumer takes is the one its producer put in the same launch (never a stale one from
the previous launch); every word a consumer needs has exactly one producer; the tag never
repeats between consecutive launches (also across the 2^32 wrap); a producer that never runs
makes every waiting group give up after its poll budget, and the grid still finishes.
"""

from __future__ import annotations

import random

import pytest

WAVES = 8
COPIES = 8  # each hand-off vector is written in 8 replicas; group g reads replica g % 8
MAX_ROWS = 4
MAX_RANGES = 128
MIN_RANGE = 64
GQA = 2
D = 4  # accumulator words per partial in the simulation (the kernel: the head dim, 128)
PART = D + 2  # a partial: running max, sum, accumulator


class Workspace:
    def __init__(self, H, I, nq, rows=MAX_ROWS):
        nk = nq // GQA
        n = {1: rows * H, 2: rows * I, 3: rows * H, "b": rows * nq * D,
             "a": rows * MAX_RANGES * nk * GQA * PART}
        self.ex = {b: [[(0, None)] * n[b] for _ in range(COPIES)] for b in n}
        self.ctl = [0, 0, 0]  # tag base, finished groups, error

    def put(self, buf, idx, word):
        for c in range(COPIES):
            self.ex[buf][c][idx] = word


def tag_of(ctl0: int) -> int:
    return ctl0 + 1  # never 0: the base stays in [0, 2^32 - 2]


def advance(ctl0: int) -> int:
    return 0 if ctl0 >= 0xFFFFFFFE else ctl0 + 1


def attn_plan(ctx, M, grid):
    """(Q, R) as the kernel's attn_plan: Q >= MIN_RANGE tokens, at most grid // M ranges per
    row and MAX_RANGES, a multiple of 16; R = ceil(longest context / Q)."""
    mx = max(ctx[:M])
    per = grid // M
    q = max(MIN_RANGE, -(-mx // per), -(-mx // MAX_RANGES))
    q = (q + 15) & ~15
    return q, -(-mx // q)


def part_word(m, j, h, g, nk):
    return (((m * MAX_RANGES + j) * nk + h) * GQA + g) * PART


def attention(ws, w, M, nq, ctx, grid, launch, log):
    """Workgroup w's attention range and, for the last M nq workgroups, a merge."""
    nk = nq // GQA
    tag = tag_of(ws.ctl[0])
    Q, R = attn_plan(ctx, M, grid)
    assert M * R <= grid and R <= MAX_RANGES
    if w < M * R:
        m, j = divmod(w, R)
        if j * Q < ctx[m]:
            for h in range(nk):
                for g in range(GQA):
                    for k in range(PART):
                        ws.put("a", part_word(m, j, h, g, nk) + k, (tag, ("p", launch, m, j, h, g, k)))
        yield
    i = grid - 1 - w
    if 0 <= i < M * nq:
        m, qh = divmod(i, nq)
        h, g = divmod(qh, GQA)
        np_ = -(-ctx[m] // Q)
        idx = [part_word(m, p, h, g, nk) + k for p in range(np_) for k in range(PART)]
        got = yield ("take", "a", idx)
        if got is None:
            return False
        log.append(("exa", (m, h, g, np_), got))
        for d in range(D):
            ws.put("b", m * nq * D + qh * D + d, (tag, ("b", launch, m, qh, d)))
    return True


def mlp_group(ws, w, M, H, I, groups, last, launch, log, nq):
    tag = tag_of(ws.ctl[0])
    C = I // groups
    yield
    got = yield ("take", "b", list(range(M * nq * D)))
    if got is None:
        return
    log.append(("exb", w, got))
    for wave in range(WAVES):
        for m in range(M):
            ws.put(1, m * H + 8 * w + wave, (tag, ("o", launch, m, 8 * w + wave)))
    got = yield ("take", 1, [m * H + k for m in range(M) for k in range(H)])
    if got is None:
        return
    log.append(("ex1", w, got))
    for m in range(M):
        for j in range(C):
            ws.put(2, m * I + C * w + j, (tag, ("a", launch, m, C * w + j)))
    got = yield ("take", 2, [m * I + k for m in range(M) for k in range(I)])
    if got is None:
        return
    log.append(("ex2", w, got))
    for wave in range(WAVES):
        for m in range(M):
            ws.put(3, m * H + 8 * w + wave, (tag, ("d", launch, m, 8 * w + wave)))
    if last:
        got = yield ("take", 3, [m * H + k for m in range(M) for k in range(H)])
        if got is None:
            return
        log.append(("ex3", w, got))


def head_group(ws, hh, M, H, mlp, launch, log):
    tag = tag_of(ws.ctl[0])
    yield
    if mlp:
        got = yield ("take", 1, [m * H + k for m in range(M) for k in range(H)])
        if got is None:
            return
        log.append(("ex1h", hh, got))
        got = yield ("take", 3, [m * H + k for m in range(M) for k in range(H)])
        if got is None:
            return
        log.append(("ex3h", hh, got))


def workgroup(ws, idx, role, M, H, I, nq, groups, grid, mlp, last, ctx, launch, log):
    if mlp:
        ok = yield from attention(ws, idx, M, nq, ctx, grid, launch, log)
        if not ok:
            return
    if role == "mlp":
        yield from mlp_group(ws, idx, M, H, I, groups, last, launch, log, nq)
    else:
        yield from head_group(ws, idx - groups, M, H, mlp, launch, log)


def run_launch(ws, H, I, M, nq, mlp, last, launch, rng, ctx, spin_limit=10**9, dead=None,
               late=()):
    """Runs one launch to completion with a random interleaving; returns the take log."""
    heads = nq + 2 * (nq // GQA)
    groups = H // 8 if mlp else 0
    grid = groups + (0 if last else heads)
    assert not mlp or M * nq <= grid  # the host's check: a merge workgroup per query head
    log = []
    # the workgroup index of each generator (MLP groups first, then head groups)
    gens = []
    for w in range(grid):
        role = "mlp" if w < groups else "head"
        gens.append((role, w, workgroup(ws, w, role, M, H, I, nq, groups, grid, mlp, last, ctx,
                                        launch, log)))
    state = {}
    for i, (_, _, g) in enumerate(gens):
        state[i] = {"gen": g, "req": None, "spins": 0, "done": False, "started": False}
    tag_at_start = {}
    steps = 0
    while not all(s["done"] for s in state.values()):
        steps += 1
        assert steps < 10**7, "schedule does not progress"
        live = [i for i, s in state.items() if not s["done"] and i != dead]
        if not live:
            break
        i = rng.choice(live)
        if i in late and steps < 200:
            continue
        s = state[i]
        g = s["gen"]
        try:
            if not s["started"]:
                s["started"] = True
                tag_at_start[i] = tag_of(ws.ctl[0])
                s["req"] = next(g)
                s["req"] = g.send(None) if s["req"] is None else s["req"]
                continue
            req = s["req"]
            if req is None:
                s["req"] = g.send(None)
                continue
            _, buf, idx = req
            copy = i % COPIES  # the generator index is the workgroup index
            words = [ws.ex[buf][copy][j] for j in idx]
            if all(t == tag_at_start[i] for t, _ in words):
                s["spins"] = 0
                s["req"] = g.send([v for _, v in words])
            else:
                s["spins"] += 1
                if s["spins"] > spin_limit:
                    ws.ctl[2] |= 1
                    s["req"] = g.send(None)
        except StopIteration:
            s["done"] = True
            ws.ctl[1] += 1
            if ws.ctl[1] == grid:  # the last finisher advances the tag base
                ws.ctl[1] = 0
                ws.ctl[0] = advance(ws.ctl[0])
    if dead is not None:  # the dead group finishes last, without doing anything
        ws.ctl[1] += 1
        if ws.ctl[1] == grid:
            ws.ctl[1] = 0
            ws.ctl[0] = advance(ws.ctl[0])
    assert len(set(tag_at_start.values())) == 1  # every group read the same tag
    return log


def check_log(log, launch, M, H, I, nq=4):
    for kind, key, got in log:
        if kind == "exa":
            m, h, g, np_ = key
            want = [("p", launch, m, p, h, g, k) for p in range(np_) for k in range(PART)]
        elif kind == "exb":
            want = [("b", launch, m, qh, d) for m in range(M) for qh in range(nq) for d in range(D)]
        elif kind.startswith("ex1"):
            want = [("o", launch, m, k) for m in range(M) for k in range(H)]
        elif kind == "ex2":
            want = [("a", launch, m, k) for m in range(M) for k in range(I)]
        else:
            want = [("d", launch, m, k) for m in range(M) for k in range(H)]
        assert got == want, kind


@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("mode", ["layer", "last", "embed"])
def test_schedule_completes_with_fresh_values(M, mode):
    """A small geometry with the kernel's ratios (H / 8 MLP groups, C = I / (H / 8), n_q =
    2 n_k), several launches in a row on one workspace with contexts that grow and shrink
    between launches (rows without context, ranges that end inside a row), random
    interleavings, some groups starting late."""
    H, I, nq = 128, 384, 4
    rng = random.Random(M * 31 + len(mode))
    ws = Workspace(H, I, nq)
    for launch in range(5):
        ctx = [rng.choice([0, 1, 63, 64, 65, 200, 700]) for _ in range(M)]
        if max(ctx) == 0:
            ctx[0] = 5
        late = set(rng.sample(range(H // 8), 2))
        log = run_launch(ws, H, I, M, nq, mode != "embed", mode == "last", launch, rng, ctx,
                         late=late)
        check_log(log, launch, M, H, I, nq)
        if mode != "embed":
            merges = [k for kind, k, _ in log if kind == "exa"]
            assert len(merges) == M * nq
            assert sum(kind == "exb" for kind, _, _ in log) == H // 8
        assert ws.ctl[2] == 0 and ws.ctl[1] == 0 and ws.ctl[0] == launch + 1


@pytest.mark.parametrize("M,grid,ctx", [(1, 160, 2048), (1, 160, 8192), (1, 160, 100000),
                                        (2, 160, 2049), (4, 40, 511), (4, 128, 3), (3, 37, 9000)])
def test_attention_ranges_cover_each_context_once(M, grid, ctx):
    """The ranges of each row tile [0, ctx) exactly, fit the grid and the partial buffer, and
    the merge reads exactly the ranges that hold tokens."""
    ctxs = [ctx] + [max(0, ctx // (m + 2)) for m in range(M - 1)]
    Q, R = attn_plan(ctxs, M, grid)
    assert Q >= MIN_RANGE and Q % 16 == 0 and M * R <= grid and R <= MAX_RANGES
    for c in ctxs:
        ranges = [(j * Q, min((j + 1) * Q, c)) for j in range(R) if j * Q < c]
        assert len(ranges) == -(-c // Q)
        toks = [t for a, b in ranges for t in range(a, b)] if c < 20000 else None
        assert toks is None or toks == list(range(c))


def test_every_needed_word_has_one_producer():
    """The producers' index maps tile ex1 / ex2 / ex3 exactly (Qwen3-0.6B geometry)."""
    H, I = 1024, 3072
    groups = H // 8
    C = I // groups
    ex1 = [8 * w + wave for w in range(groups) for wave in range(WAVES)]
    ex2 = [C * w + j for w in range(groups) for j in range(C)]
    assert sorted(ex1) == list(range(H)) and sorted(ex2) == list(range(I))
    # gate_up rows of a group: 16 per pass (8 wavefronts x 2 halves), gate then up
    passes = 2 * C // 16
    rows = []
    for w in range(3):
        for p in range(passes):
            for wave in range(WAVES):
                for half in range(2):
                    r = 16 * p + 2 * wave + half
                    rows.append(C * w + r if r < C else I + C * w + (r - C))
    assert len(set(rows)) == len(rows) == 3 * 2 * C
    # the head groups' residual shares tile the hidden size
    heads = 32
    share = H // heads
    assert sorted(k for hh in range(heads) for k in range(hh * share, (hh + 1) * share)) == list(range(H))


def test_tag_never_repeats_across_wrap():
    base = 0xFFFFFFFD
    tags = []
    for _ in range(5):
        tags.append(tag_of(base))
        base = advance(base)
    assert all(t != 0 and t <= 0xFFFFFFFF for t in tags)
    assert all(a != b for a, b in zip(tags, tags[1:]))


def test_a_missing_producer_makes_waits_give_up():
    """One MLP group never runs: the groups waiting on its words give up after their poll
    budget, the error word is set, and every other group still finishes (the grid drains)."""
    H, I, nq, M = 64, 192, 4, 2
    ws = Workspace(H, I, nq)
    rng = random.Random(5)
    run_launch(ws, H, I, M, nq, True, False, 0, rng, [300, 40], spin_limit=50, dead=3)
    assert ws.ctl[2] == 1 and ws.ctl[1] == 0 and ws.ctl[0] == 1
