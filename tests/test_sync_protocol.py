"""CPU model of the single launch's cross-workgroup protocol (csrc/sdv_attn.hip, fused_kernel).

Workgroups are coroutines that yield at every access to the synchronisation area; a seeded
scheduler interleaves them at random, can hold one workgroup back until the others have given
up on it (a late publisher), and runs calls one after another as a stream does.  The model
follows the kernel's rules step by step:

* statistics are (value, tag) words; a reader takes one only when its tag is the call's own;
* a partial word is "written" when non-zero: an item zeroes its own partial slot at the start
  and (once those stores completed) publishes its statistics; it polls the group's statistics,
  publishes its partial; the owner of an output slice, having taken every item's statistics of
  this call, polls every item's slice, sums it in item order, then clears a share of the
  statistics;
* a wait is bounded: an expired wait makes the affected outputs NaN, counts a failure, skips
  the clears, and -- for a graph-recorded call -- poisons the area; a graph-recorded call reads
  the poison with its statistics poll and, when set, ends with NaN outputs, counted.

Every word records which call wrote it, and a reader asserts that a word it accepts came
from its own call: that is the claim "no stale entry survives into a later call".  Planted
mistakes (no clears, tags reused by eager calls, a partial slot not zeroed first, ignoring the
poison) break it, so the model has teeth.
"""
from __future__ import annotations

import math
import random

import pytest

GRAPH_BIT = 0x80000000


class StaleRead(AssertionError):
    pass


class Area:
    """The workspace's synchronisation area: word slots plus the failure count and poison."""

    def __init__(self):
        self.words: dict = {}   # key -> (value, tag, writer call id)
        self.fail = 0
        self.poison = 0

    def reset(self):
        self.__init__()


class Call:
    """One single-launch call: `groups` groups of `items` items, `chunks` output chunks per group."""

    _ids = 0

    def __init__(self, groups, items, chunks, tag, seed_inputs, spin_limit=10_000, clears=True,
                 honour_poison=True, zero_slot=True):
        Call._ids += 1
        self.id = Call._ids
        self.groups, self.items, self.chunks = groups, items, chunks
        self.tag = tag
        self.graph = bool(tag & GRAPH_BIT)
        self.spin_limit = spin_limit
        self.clears = clears
        self.honour_poison = honour_poison
        self.zero_slot = zero_slot
        rng = random.Random(seed_inputs)
        # item statistic and per-chunk contribution of every (group, item): the expected output of
        # chunk o of group g is sum_i contrib(g, i, o) * combine(stats of g)
        self.stat = [[rng.randint(1, 9) for _ in range(items)] for _ in range(groups)]
        self.contrib = [[[rng.randint(1, 9) for _ in range(chunks)] for _ in range(items)] for _ in range(groups)]
        self.out = [[None] * chunks for _ in range(groups)]

    def expected(self, g, o):
        m = sum(self.stat[g])
        return sum(self.contrib[g][i][o] * m for i in range(self.items))

    # ------------------------------------------------------------------ one workgroup
    def workgroup(self, area: Area, g: int, c: int):
        """Coroutine of item c of group g (mirrors fused_kernel's order of accesses)."""
        n, tag = self.items, self.tag
        per = -(-self.chunks // n)
        lo, hi = c * per, min(self.chunks, c * per + per)
        nown = -(-self.chunks // per)
        item = g * n + c
        if self.zero_slot:                             # zero the own partial slot first ...
            for o in range(self.chunks):
                area.words[("part", item, o)] = (0, 0, 0)
                yield
        # ... those stores complete (vmcnt(0)) before the statistics are published
        area.words[("stat", item)] = (self.stat[g][c], tag, self.id)
        yield
        fail = False
        poison = area.poison if self.graph else 0      # read with the statistics poll
        # group statistics: poll every item of the group
        m = 0
        for i in range(n):
            spins = 0
            while True:
                w = area.words.get(("stat", g * n + i))
                if w is not None and w[1] == tag:
                    if w[2] != self.id and not (poison and self.honour_poison):
                        raise StaleRead(f"call {self.id} took a statistic written by call {w[2]}")
                    m += w[0]
                    break
                spins += 1
                if spins >= self.spin_limit:
                    fail, m = True, math.nan
                    break
                yield
            if fail:
                break
        if poison and self.honour_poison:
            fail, m = True, math.nan
        # partial of this item: one word per output chunk (a partial word is never 0)
        for o in range(self.chunks):
            area.words[("part", item, o)] = (self.contrib[g][c][o] * m, -1, self.id)
            yield
        # owner: poll the slice of every item's partial
        got = {}
        for i in range(n):
            for o in range(lo, hi):
                spins = 0
                while True:
                    w = area.words.get(("part", g * n + i, o))
                    if w is not None and w[1] != 0:
                        if w[2] != self.id and not fail:
                            raise StaleRead(f"call {self.id} took a partial written by call {w[2]}")
                        got[(i, o)] = w[0]
                        break
                    spins += 1
                    if spins >= self.spin_limit:
                        fail = True
                        break
                    yield
        if fail:
            for o in range(lo, hi):
                self.out[g][o] = math.nan
            area.fail += 1
            if self.graph:
                area.poison = 1
            return
        for o in range(lo, hi):
            self.out[g][o] = sum(got[(i, o)] for i in range(n))
        if not self.clears:
            return
        if c < nown:
            for e in range(c, n, nown):
                area.words[("stat", g * n + e)] = (0, 0, 0)
                yield

    # ------------------------------------------------------------------ the whole call
    def run(self, area: Area, rng: random.Random, late: tuple | None = None):
        """Interleave every workgroup at random until all finish.  late = (g, c): that workgroup
        starts only once every other workgroup has finished (it publishes after the others gave
        up on it)."""
        pending = {(g, c): self.workgroup(area, g, c) for g in range(self.groups) for c in range(self.items)}
        held = pending.pop(late) if late is not None else None
        while pending:
            key = rng.choice(sorted(pending))
            try:
                next(pending[key])
            except StopIteration:
                del pending[key]
        if held is not None:
            for _ in held:
                pass

    def check(self, allow_nan: bool):
        """Every output is its expected value, or NaN where the call failed."""
        nans = 0
        for g in range(self.groups):
            for o in range(self.chunks):
                v = self.out[g][o]
                assert v is not None, "an output was never written"
                if isinstance(v, float) and math.isnan(v):
                    nans += 1
                    assert allow_nan, f"call {self.id}: NaN at group {g} chunk {o}"
                else:
                    assert v == self.expected(g, o), f"call {self.id}: wrong output at group {g} chunk {o}"
        return nans


class Tags:
    """The library's tag counter: fresh 31-bit tags, bit 31 for graph-recorded calls."""

    def __init__(self):
        self.n = 0

    def next(self, graph=False):
        self.n += 1
        return (self.n & ~GRAPH_BIT) | (GRAPH_BIT if graph else 0)


SHAPES = [(3, 4, 7), (2, 3, 5), (4, 2, 9), (1, 5, 3)]   # (groups, items, chunks)


@pytest.mark.parametrize("seed", range(40))
def test_normal_calls_leave_the_area_clean(seed):
    rng = random.Random(seed)
    area, tags = Area(), Tags()
    for k in range(4):
        shp = SHAPES[(seed + k) % len(SHAPES)]
        call = Call(*shp, tags.next(), seed * 100 + k)
        call.run(area, rng)
        assert call.check(allow_nan=False) == 0
        assert area.fail == 0
        assert all(w[1] == 0 for k_, w in area.words.items() if k_[0] == "stat"), \
            "a statistics word survived a normal call"


@pytest.mark.parametrize("seed", range(60))
def test_expired_eager_call_then_next_call_is_correct(seed):
    """An eager call whose waits expire (a late publisher writes after everyone gave up) leaves
    words behind; the next eager call on the area -- any shape -- ignores them and is exact."""
    rng = random.Random(seed)
    area, tags = Area(), Tags()
    shp = SHAPES[seed % len(SHAPES)]
    bad = Call(*shp, tags.next(), seed, spin_limit=rng.randint(1, 6))
    bad.run(area, rng, late=(rng.randrange(shp[0]), rng.randrange(shp[1])))
    nans = bad.check(allow_nan=True)
    assert area.fail > 0 and nans > 0, "the failure was not surfaced"
    assert area.poison == 0, "an eager call must not poison the area"
    for k in range(3):
        nxt = Call(*SHAPES[(seed + k + 1) % len(SHAPES)], tags.next(), seed * 7 + k)
        fails = area.fail
        nxt.run(area, rng)
        assert nxt.check(allow_nan=False) == 0
        assert area.fail == fails


@pytest.mark.parametrize("seed", range(40))
def test_graph_replays_poison_and_reset(seed):
    """Graph replays reuse their recorded tag: normal replays are exact (the clears); a replay
    that expires poisons the area, every graph-recorded call is then refused (NaN, counted)
    while eager calls stay exact, and a reset restores the replays."""
    rng = random.Random(seed)
    area, tags = Area(), Tags()
    shp = SHAPES[seed % len(SHAPES)]
    t_good = tags.next(graph=True)
    for r in range(3):   # the replays of one recorded call, new inputs each time
        rep = Call(*shp, t_good, seed * 10 + r)
        rep.run(area, rng)
        assert rep.check(allow_nan=False) == 0
    t_bad = tags.next(graph=True)
    bad = Call(*shp, t_bad, seed, spin_limit=1)
    bad.run(area, rng, late=(0, shp[1] - 1))
    bad.check(allow_nan=True)
    assert area.fail > 0 and area.poison == 1
    refused = Call(*shp, t_good, seed + 1)
    refused.run(area, rng)
    assert refused.check(allow_nan=True) == shp[0] * shp[2], "a poisoned graph call must write NaN everywhere"
    eager = Call(*SHAPES[(seed + 1) % len(SHAPES)], tags.next(), seed + 2)
    eager.run(area, rng)
    assert eager.check(allow_nan=False) == 0
    area.reset()
    again = Call(*shp, t_good, seed + 3)
    again.run(area, rng)
    assert again.check(allow_nan=False) == 0


# ---------------------------------------------------------------------- planted mistakes
def _find_stale(make_calls, seeds=range(80)):
    for seed in seeds:
        try:
            make_calls(seed)
        except (StaleRead, AssertionError):
            return True
    return False


def test_planted_no_clears_breaks_graph_replays():
    def run(seed):
        rng = random.Random(seed)
        area, tags = Area(), Tags()
        t = tags.next(graph=True)
        for r in range(3):
            rep = Call(*SHAPES[seed % len(SHAPES)], t, seed * 10 + r, clears=False)
            rep.run(area, rng)
            rep.check(allow_nan=False)
    assert _find_stale(run), "replays without clears should read an earlier replay's words"


def test_planted_reused_eager_tag_breaks_recovery():
    def run(seed):
        rng = random.Random(seed)
        area = Area()
        shp = SHAPES[seed % len(SHAPES)]
        bad = Call(*shp, 5, seed, spin_limit=1)
        bad.run(area, rng, late=(0, 0))
        nxt = Call(*shp, 5, seed + 1)        # same tag again: the words the late publisher left look current
        nxt.run(area, rng)
        nxt.check(allow_nan=False)
    assert _find_stale(run)


def test_planted_unzeroed_slot_breaks_recovery():
    """Without the item zeroing its partial slot first, a late publisher's partial survives
    into the next eager call and is read as current."""
    def run(seed):
        rng = random.Random(seed)
        area, tags = Area(), Tags()
        shp = SHAPES[seed % len(SHAPES)]
        bad = Call(*shp, tags.next(), seed, spin_limit=1)
        bad.run(area, rng, late=(0, 0))
        nxt = Call(*shp, tags.next(), seed + 1, zero_slot=False)
        nxt.run(area, rng)
        nxt.check(allow_nan=False)
    assert _find_stale(run)


def test_planted_ignored_poison_breaks_replays():
    def run(seed):
        rng = random.Random(seed)
        area = Area()
        shp = SHAPES[seed % len(SHAPES)]
        t = GRAPH_BIT | 3
        bad = Call(*shp, t, seed, spin_limit=1)
        bad.run(area, rng, late=(0, shp[1] - 1))
        rep = Call(*shp, t, seed + 1, honour_poison=False)
        rep.run(area, rng)
        rep.check(allow_nan=False)
    assert _find_stale(run)
