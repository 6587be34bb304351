"""CPU model of the single launch's work assignment and lane reductions (csrc/sdv_attn.hip,
fused_kernel), replayed for every size the kernel can meet:

* the static streaming loops (q.k^T blocks and p.V units): wavefront w takes items
  w, w + W, ... with two in flight, a loop over pairs and the last one or two peeled after it;
  every item is computed exactly once, from the buffer last loaded with it, and nothing past
  the end is loaded;
* the verify V ring: full rounds of SD stages in a loop, the last (up to 2 SD - 1) stages
  after it; the same properties per wavefront part;
* the output stage: each output chunk gets a group of P2 lanes (the item count rounded up to a
  power of two), the lanes load one item's chunk each (items past the group's count load
  nothing and add 0), and a butterfly of quad permutes, DPP row shifts and half-wave pairs
  leaves the group's sum in its first lane, which writes it.  The lane exchanges are modelled
  with the hardware's semantics (a row shift reads 0 past the end of its 16-lane row), and
  the check uses distinct integer weights, so a missing or doubled term fails exactly.
A planted mistake (a row shift in the wrong direction, or a loop that loads one past the end)
must fail the model.
"""
from __future__ import annotations

import pytest


# ---------------------------------------------------------------- static loops
def static_loop(nitems: int, wave: int, W: int):
    """The peeled two-buffer loop of q.k^T / p.V units: the events (op, buffer, item)."""
    ev = []
    ns = (nitems - 1 - wave) // W + 1 if wave < nitems else 0
    item = lambda s: wave + s * W
    if ns > 0:
        ev.append(("load", "a", item(0)))
        s = 0
        while s + 2 < ns:
            ev += [("load", "b", item(s + 1)), ("compute", "a", item(s)),
                   ("load", "a", item(s + 2)), ("compute", "b", item(s + 1))]
            s += 2
        if s + 1 < ns:
            ev += [("load", "b", item(s + 1)), ("compute", "a", item(s)), ("compute", "b", item(s + 1))]
        else:
            ev.append(("compute", "a", item(s)))
    return ev


def check_events(ev, valid):
    """Every computed item was the last one loaded into its buffer; no load outside `valid`;
    at most two loads outstanding (loaded, not yet computed)."""
    buf, pending, computed = {}, set(), []
    for op, b, it in ev:
        if op == "load":
            assert it in valid, f"load of {it} outside the items"
            buf[b] = it
            pending.add(it)
            assert len(pending) <= 2
        else:
            assert buf.get(b) == it, f"computes {it} from a buffer holding {buf.get(b)}"
            pending.discard(it)
            computed.append(it)
    return computed


@pytest.mark.parametrize("W", [8, 16])
def test_static_loops_cover_every_item_once(W):
    for n in range(0, 300):
        seen = []
        for w in range(W):
            seen += check_events(static_loop(n, w, W), set(range(n)))
        assert sorted(seen) == list(range(n)), n


def test_planted_loop_past_the_end_fails():
    def bad_loop(n, wave, W):  # reloads unconditionally, as a counter-claimed loop does
        ev = static_loop(n, wave, W)
        return ev + [("load", "a", wave + n * W)] if ev else ev
    with pytest.raises(AssertionError):
        for w in range(8):
            check_events(bad_loop(100, w, 8), set(range(100)))


# ---------------------------------------------------------------- verify V ring
def ring_schedule(nstage: int, SD: int):
    ev = [("load", i, i) for i in range(SD) if i < nstage]
    st0 = 0
    while st0 + 2 * SD <= nstage:
        for i in range(SD):
            ev += [("compute", i, st0 + i), ("load", i, st0 + i + SD)]
        st0 += SD
    for i in range(SD):
        if st0 + i < nstage:
            ev.append(("compute", i, st0 + i))
            if st0 + i + SD < nstage:
                ev.append(("load", i, st0 + i + SD))
    for i in range(SD):
        if st0 + SD + i < nstage:
            ev.append(("compute", i, st0 + SD + i))
    return ev


@pytest.mark.parametrize("SD", [1, 2, 3, 6])
def test_verify_ring_covers_every_stage_once(SD):
    for n in range(0, 80):
        buf, done = {}, []
        for op, slot, st in ring_schedule(n, SD):
            if op == "load":
                assert 0 <= st < n, "load past the part"
                buf[slot] = st
            else:
                assert buf.get(slot) == st
                done.append(st)
        assert done == list(range(n)), (SD, n)


# ---------------------------------------------------------------- output butterfly
def xor_low(vals, X, right=False):
    """lane_xor_low<X>: quad permutes for X = 1, 2 (every lane valid); for X = 4, 8 the DPP row
    shift left (lane i reads lane i + X of its 16-lane row, 0 past the row's end).  right: the
    row shift the other way (lane i reads lane i - X), a planted mistake."""
    out = []
    for i in range(64):
        if X in (1, 2):
            out.append(vals[i ^ X])
        else:
            j = i - X if right else i + X
            out.append(vals[j] if 0 <= j < 64 and j // 16 == i // 16 else 0)
    return out


def pair16(vals):
    """lane_pair<16>: both lanes of rows 2k and 2k+1 get (lower, upper)."""
    return [(vals[i & ~16], vals[i | 16]) for i in range(64)]


def butterfly(vals, P2, right=False):
    f = list(vals)
    if P2 > 1:
        f = [a + b for a, b in zip(f, xor_low(f, 1))]
    if P2 > 2:
        f = [a + b for a, b in zip(f, xor_low(f, 2))]
    if P2 > 4:
        f = [a + b for a, b in zip(f, xor_low(f, 4, right))]
    if P2 > 8:
        f = [a + b for a, b in zip(f, xor_low(f, 8, right))]
    if P2 > 16:
        f = [lo + hi for lo, hi in pair16(f)]
    return f


def owner_stage(nvq: int, w: int, NTHR: int = 512, loads: int = 4, right: bool = False):
    """Output chunk o -> the value its group's first lane writes; also every (item, chunk)
    load, to check coverage.  Item cc's chunk o carries the weight 1000 * (cc + 1) + o."""
    P2 = 1
    while P2 < nvq:
        P2 *= 2
    nsl = w * P2
    written, loaded = {}, []
    for e0 in range(0, nsl, NTHR * loads):
        for r in range(loads):
            if e0 + r * NTHR >= nsl:
                break
            for wave in range(NTHR // 64):
                vals = []
                for lane in range(64):
                    e = e0 + r * NTHR + wave * 64 + lane
                    o, cc = divmod(e, P2)
                    act = e < nsl and cc < nvq
                    if act:
                        loaded.append((cc, o))
                    vals.append(1000 * (cc + 1) + o if act else 0)
                f = butterfly(vals, P2, right)
                for lane in range(64):
                    e = e0 + r * NTHR + wave * 64 + lane
                    o, cc = divmod(e, P2)
                    if cc == 0 and e < nsl:
                        assert o not in written, "chunk written twice"
                        written[o] = f[lane]
    return written, loaded


@pytest.mark.parametrize("nvq", list(range(1, 33)))
def test_output_butterfly_sums_each_chunk_once(nvq):
    for w in (0, 1, 4, 6, 30, 48, 240):
        written, loaded = owner_stage(nvq, w)
        assert sorted(loaded) == sorted((cc, o) for cc in range(nvq) for o in range(w))
        assert sorted(written) == list(range(w))
        for o, v in written.items():
            assert v == sum(1000 * (cc + 1) + o for cc in range(nvq)), (nvq, w, o)


def test_planted_row_shift_direction_fails():
    """A row shift to the right would hand the group's first lane zeros or another chunk's lanes."""
    with pytest.raises(AssertionError):
        for nvq in (5, 9, 16):
            written, _ = owner_stage(nvq, 6, right=True)
            for o, v in written.items():
                assert v == sum(1000 * (cc + 1) + o for cc in range(nvq))


# ---------------------------------------------------------------- per-sequence item plan
def seq_plan(lens, L, KV, maxblk, grid, bisect=True):
    """fused_kernel's item plan for a batch with per-sequence lengths: workgroup -> (group, c,
    items of the group, blocks of the group, first item) or None past the plan, replayed with
    the kernel's integer arithmetic: ceil(blocks / S) items per sequence (at most 32, at most one
    per block, one for an empty sequence) for the smallest S in [1, maxblk] whose items fit the
    grid.  bisect=False: a plain proportional share instead (a planted mistake)."""
    B = len(lens)
    blk = [-(-t // 16) for t in lens]
    gs = L * KV

    def items_for(sz):
        return [1 if t == 0 else min(32, b, -(-b // sz)) for t, b in zip(lens, blk)]

    if bisect:
        lo, hi = 1, maxblk
        while lo < hi:
            mid = (lo + hi) // 2
            if gs * sum(items_for(mid)) <= grid:
                hi = mid
            else:
                lo = mid + 1
        items = items_for(lo)
    else:
        total = gs * sum(blk)
        items = [1 if t == 0 else min(32, b, 1 + ((grid - gs * B) * gs * b) // total) for t, b in zip(lens, blk)]
    excl = [sum(items[:i]) for i in range(B)]
    per_layer = KV * sum(items)
    out = []
    for item in range(grid):
        li = item // per_layer
        if li >= L:
            out.append(None)
            continue
        r = item - li * per_layer
        bs = next(b for b in range(B) if KV * excl[b] <= r < KV * (excl[b] + items[b]))
        h, c = divmod(r - KV * excl[bs], items[bs])
        out.append(((li * B + bs) * KV + h, c, items[bs], blk[bs], item - c))
    return out


def host_shape(max_len, G, cap):
    """The host planner's items per group (base) and LDS width in blocks (maxblk)."""
    gb = -(-max_len // 16)
    base = min(32, gb, cap // G)
    return base, -(-gb // base)


def check_seq_plan(lens, L, KV, cap, bisect=True):
    G = L * len(lens) * KV
    base, maxblk = host_shape(max(lens), G, cap)
    plan = seq_plan(lens, L, KV, maxblk, cap, bisect)
    assert sum(e is not None for e in plan) <= cap
    seen = {}
    for item, e in enumerate(plan):
        if e is None:
            continue
        grp, c, n_g, gbg, item0 = e
        seen.setdefault(grp, []).append((c, item, n_g, gbg, item0))
    assert sorted(seen) == list(range(G)), "every group has items"
    for grp, its in seen.items():
        its.sort()
        n_g, gbg = its[0][2], its[0][3]
        assert [c for c, *_ in its] == list(range(n_g)), "items of a group: c = 0 .. n_g-1"
        assert [i for _, i, *_ in its] == list(range(its[0][4], its[0][4] + n_g)), "contiguous"
        covered = 0
        for c, *_ in its:
            lo, hi = c * gbg // n_g, (c + 1) * gbg // n_g
            assert lo == covered
            covered = hi
            assert hi - lo <= maxblk, f"item of {hi - lo} blocks over the LDS width {maxblk}"
            assert gbg == 0 or hi - lo >= 1, "empty item in a non-empty sequence"
        assert covered == gbg
    return plan


@pytest.mark.parametrize("seed", range(60))
def test_per_sequence_item_plan(seed):
    import random
    rng = random.Random(seed)
    B = rng.randint(2, 64)
    L = rng.choice([1, 1, 2, 4])
    KV = rng.choice([1, 2])
    cap = rng.choice([224, 256, 512])
    if L * B * KV > cap:
        B = max(2, cap // (L * KV))
    top = rng.choice([17, 2048, 8192, 32768])
    lens = [rng.choice([0, 1, rng.randint(1, top), top]) for _ in range(B)]
    if max(lens) == 0:
        lens[0] = 5
    check_seq_plan(lens, L, KV, cap)


def test_per_sequence_plan_config4_layer():
    """Config 4's per-layer call: the longest items shrink from 512 blocks."""
    import random
    rng = random.Random(41)
    lens = [2048, 32768] + [rng.randint(2048, 32768) for _ in range(30)]
    plan = check_seq_plan(lens, 1, 2, 256)
    longest = max(-(-e[3] // e[2]) for e in plan if e is not None)
    assert longest < 512


def test_planted_plain_proportional_share_overflows_lds():
    """A plain proportional share gives a sequence just short of a share threshold too few
    items, and one of them overflows the LDS width."""
    lens = [32768] * 31 + [30000]
    with pytest.raises(AssertionError):
        check_seq_plan(lens, 1, 2, 256, bisect=False)
