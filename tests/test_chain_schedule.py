"""CPU simulation of the decode chain's hand-off schedule (llm-serving-engine_amd/csrc/
decode_chain.hip), run before the kernel ever runs on a GPU.

The kernel's workgroups are restated as Python generators that perform the same sequence of
hand-off operations with the same index formulas: MLP group w puts o_proj rows 8w..8w+7 into
ex1, takes all of ex1, puts silu * up channels [C w, C (w + 1)) into ex2, takes all of ex2, puts
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


class Workspace:
    def __init__(self, H, I, rows=4):
        n = {1: rows * H, 2: rows * I, 3: rows * H}
        self.ex = {b: [[(0, None)] * n[b] for _ in range(COPIES)] for b in n}
        self.ctl = [0, 0, 0]  # tag base, finished groups, error

    def put(self, buf, idx, word):
        for c in range(COPIES):
            self.ex[buf][c][idx] = word


def tag_of(ctl0: int) -> int:
    return ctl0 + 1  # never 0: the base stays in [0, 2^32 - 2]


def advance(ctl0: int) -> int:
    return 0 if ctl0 >= 0xFFFFFFFE else ctl0 + 1


def mlp_group(ws, w, M, H, I, groups, last, launch, log):
    tag = tag_of(ws.ctl[0])
    C = I // groups
    yield
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


def run_launch(ws, H, I, M, heads, mlp, last, launch, rng, spin_limit=10**9, dead=None,
               late=()):
    """Runs one launch to completion with a random interleaving; returns the take log."""
    groups = H // 8 if mlp else 0
    log = []
    # the workgroup index of each generator (MLP groups first, then head groups)
    gens = []
    for w in range(groups):
        gens.append(("mlp", w, mlp_group(ws, w, M, H, I, groups, last, launch, log)))
    for hh in range(0 if last else heads):
        gens.append(("head", hh, head_group(ws, hh, M, H, mlp, launch, log)))
    grid = len(gens)
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


def check_log(log, launch, M, H, I):
    for kind, _, got in log:
        if kind.startswith("ex1"):
            want = [("o", launch, m, k) for m in range(M) for k in range(H)]
        elif kind == "ex2":
            want = [("a", launch, m, k) for m in range(M) for k in range(I)]
        else:
            want = [("d", launch, m, k) for m in range(M) for k in range(H)]
        assert got == want, kind


@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("mode", ["layer", "last", "embed"])
def test_schedule_completes_with_fresh_values(M, mode):
    """A small geometry with the kernel's ratios (H / 8 MLP groups, C = I / (H / 8)), several
    launches in a row on one workspace, random interleavings, some groups starting late."""
    H, I, heads = 64, 192, 6
    rng = random.Random(M * 31 + len(mode))
    ws = Workspace(H, I)
    for launch in range(4):
        late = set(rng.sample(range(H // 8), 2))
        log = run_launch(ws, H, I, M, heads, mode != "embed", mode == "last", launch, rng,
                         late=late)
        check_log(log, launch, M, H, I)
        assert ws.ctl[2] == 0 and ws.ctl[1] == 0 and ws.ctl[0] == launch + 1


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
    H, I, heads, M = 64, 192, 6, 2
    ws = Workspace(H, I)
    rng = random.Random(5)
    run_launch(ws, H, I, M, heads, True, False, 0, rng, spin_limit=50, dead=3)
    assert ws.ctl[2] == 1 and ws.ctl[1] == 0 and ws.ctl[0] == 1
