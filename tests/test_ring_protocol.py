"""Interleaving model of the attention kernel's LDS copy ring (CPU only).

The tile kernel (leanselect_amd/csrc/ls_attention.hip, ring protocol around
lines 401-610) streams the tile's union pages through 4 LDS stages.  Union
page u uses stage u % 4.  Shared state: ``s_next`` (next page to claim),
``s_done[st] = (page << 8) | waves done with it`` and the ready token
``s_rdy[st] = page + 1``, which a page's copy writes with its final load.
Waves 0..3 copy pages 0..3 at the start; afterwards only a waiting wave copies:
at page ``ui`` it may claim ``nx = s_next`` when ``nx <= ui + 3`` and the
stage's previous page ``nx - 4`` has been finished by every wave that needs
it (tag and count match), by a compare-and-swap on ``s_next``; it then resets
``s_done`` to ``nx << 8`` and issues the copy without waiting for it.  A wave
computes a page once its token is there and then adds one to ``s_done``.

The model runs the waves' shared-memory steps and the copies' landings in
random orders and checks, over many random tile plans:
- safety: no copy into a stage is issued while a wave still needs or reads the
  page in it, and a wave only reads a stage that holds its page;
- liveness: every wave finishes (the kernel's bounded wait never expires).
It also shows what the protocol rests on: with the token allowed to land
before the page data (loads of one wave landing out of order), or with the
claim ignoring the stage's tag, the model finds a violation.
"""
import random

import pytest

STAGES = 4


class Violation(Exception):
    pass


def run_ring(need, seed, *, token_in_order=True, check_tag=True, max_ticks=200000):
    """Simulate one tile.  ``need[w]`` is the sorted list of union pages wave
    ``w`` computes.  Returns the number of ticks; raises Violation."""
    rng = random.Random(seed)
    n_waves = len(need)
    n_union = 1 + max((p for ps in need for p in ps), default=-1)
    uneed = [sum(1 for ps in need if u in ps) for u in range(n_union)]
    s_next = STAGES
    s_done = [0] * STAGES
    s_rdy = [0] * STAGES
    stage_page = [None] * STAGES   # page whose data the stage holds
    in_flight = []                 # [stage, page, data_landed]
    readers = [set() for _ in range(STAGES)]   # waves reading the stage now
    finished = {u: 0 for u in range(n_union)}

    def issue_copy(u):
        st = u % STAGES
        prev = u - STAGES
        if prev >= 0 and finished[prev] != uneed[prev]:
            raise Violation(f"copy of page {u} issued while page {prev} still needed")
        if readers[st]:
            raise Violation(f"copy of page {u} issued while stage {st} is read")
        s_done[st] = u << 8
        in_flight.append([st, u, False])

    def wave(w):
        # Generator: one yield per shared-memory step.
        if w < STAGES and w < n_union:
            issue_copy(w)
            yield
        for ui in need[w]:
            st = ui % STAGES
            while s_rdy[st] != ui + 1:
                yield
                nx = s_next
                yield
                if nx >= n_union or nx > ui + STAGES - 1:
                    continue
                prev = nx - STAGES
                done = s_done[nx % STAGES]
                yield
                want_ok = (done == ((prev << 8) | uneed[prev])) if check_tag \
                    else ((done & 0xff) == uneed[prev])
                if not want_ok:
                    continue
                if s_next != nx:      # compare-and-swap lost
                    continue
                s_next_set(nx + 1)
                for _ in range(rng.randint(1, 6)):  # the claim won; the reset store is still to come
                    yield
                issue_copy(nx)
                yield
            # compute: a few read steps of the stage
            readers[st].add(w)
            for _ in range(rng.randint(1, 3)):
                if stage_page[st] != ui:
                    raise Violation(f"wave {w} reads stage {st} holding {stage_page[st]}, not {ui}")
                yield
            readers[st].discard(w)
            s_done[st] += 1
            finished[ui] += 1
            yield

    def s_next_set(v):
        nonlocal s_next
        s_next = v

    waves = {w: wave(w) for w in range(n_waves)}
    ticks = 0
    while waves or in_flight:
        ticks += 1
        if ticks > max_ticks:
            raise Violation("no progress: a wait would not end")
        choices = list(waves.keys()) + [("copy", i) for i in range(len(in_flight))]
        c = rng.choice(choices)
        if isinstance(c, tuple):
            st, u, landed = in_flight[c[1]]
            if not token_in_order and rng.random() < 0.5 and s_rdy[st] != u + 1:
                s_rdy[st] = u + 1          # the token may overtake the data
                continue
            if not landed:
                stage_page[st] = u
                in_flight[c[1]][2] = True
                if token_in_order:
                    continue
            s_rdy[st] = u + 1
            if in_flight[c[1]][2]:
                in_flight.pop(c[1])
            continue
        try:
            next(waves[c])
        except StopIteration:
            del waves[c]
    return ticks


def random_need(rng, n_waves=8, n_union=None, p=0.35):
    n_union = n_union or rng.randint(1, 80)
    need = [[] for _ in range(n_waves)]
    for u in range(n_union):
        ws = [w for w in range(n_waves) if rng.random() < p] or [rng.randrange(n_waves)]
        for w in ws:
            need[w].append(u)
    return need


@pytest.mark.parametrize("p", [0.1, 0.35, 0.9])
def test_ring_is_safe_and_always_drains(p):
    rng = random.Random(1234)
    for trial in range(150):
        need = random_need(rng, p=p)
        run_ring(need, seed=trial)


def test_ring_edge_shapes():
    run_ring([[0]] + [[] for _ in range(7)], seed=0)           # one page
    run_ring([[0, 1, 2]] + [[] for _ in range(7)], seed=1)     # fewer pages than stages
    run_ring([list(range(60))] + [[] for _ in range(7)], seed=2)  # one busy wave
    run_ring([[u] for u in range(8)], seed=3)                  # one page per wave
    run_ring([list(range(40)) for _ in range(8)], seed=4)      # every wave every page


def test_model_catches_a_token_landing_before_its_data():
    rng = random.Random(7)
    found = False
    for trial in range(300):
        try:
            run_ring(random_need(rng, p=0.5), seed=trial, token_in_order=False)
        except Violation:
            found = True
            break
    assert found, "the in-order landing of a wave's loads is what keeps readers on fresh data"


def test_model_catches_a_claim_that_ignores_the_stage_tag():
    # Every page needed by one wave: a stale count of the stage's older page
    # then matches, and only the tag tells the pages apart.
    rng = random.Random(8)
    found = False
    for trial in range(400):
        n_union = rng.randint(12, 60)
        need = [[] for _ in range(8)]
        for u in range(n_union):
            need[rng.randrange(8)].append(u)
        try:
            run_ring(need, seed=trial, check_tag=False)
        except Violation:
            found = True
            break
    assert found, "without the page tag a stale count lets a copy overwrite a live stage"
