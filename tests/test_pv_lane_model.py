"""CPU model of the three-launch p.V kernel's lane indexing (csrc/sdv_attn.hip, pv_kernel,
pv_load and pv_compute), run on the shapes of the multi-layer GPU tests.

Each workgroup (chunk c, KV head, sequence) has 4 wavefronts; wavefront w takes blocks
[blk0, blk0 + nb) of its sequence, lane l < nb holds the page id of block blk0 + l, and a
stage of 4 blocks gives lane group g the block 4*st + g, fetched with a lane shuffle from
lane 4*st + g (lane 0 past the wavefront).  A stage is "full" when all its blocks lie below
T and exist; otherwise its slots that are not tokens of the sequence are sanitized (codes,
scales to 0, scores to -inf).  The model replays exactly that indexing and checks, for every
slot that reaches the MFMA with a score that is not -inf:

* it is a token of the sequence (position < T) in a block with a valid page id, and the page
  is the one the block table names for that block;
* its score was written by q.k^T (q.k^T writes whole blocks below ceil(T/16) for every row);
* the score load stays inside the workspace row (score_stride), the shuffle source lane is
  inside the wavefront, and every stage that holds a non-token slot is sanitized.

The planner's chunk sizes follow make_plan (kWaves = 4 wavefronts per workgroup, page
blocks per wavefront doubling with the problem size up to 64).  A planted mistake (no
sanitizing of a partial stage) must fail the model.
"""
from __future__ import annotations

import random

import pytest

K_WAVES, K_WAVE, K_BLOCK, QK_SCORE_TOKENS = 4, 64, 16, 128


def plan(L, B, KV, S, G, tmax):
    """Chunking of make_plan for one row-tile group per KV head (decode and short verify)."""
    r = G * S
    nt = 1 if r <= 16 else 2 if r <= 32 else 3 if r <= 48 else 4
    nrg = -(-r // (16 * nt))
    units = L * B * KV * nrg
    blocks = units * (-(-tmax // K_BLOCK))
    qb, qb_max = 1, max(1, QK_SCORE_TOKENS // (K_BLOCK * nt))
    while qb < qb_max and blocks > K_WAVES * qb * 1024:
        qb *= 2
    pb = 4
    while pb < K_WAVE and blocks > K_WAVES * pb * 512:
        pb *= 2
    qk_chunk = K_WAVES * qb * K_BLOCK
    pv_chunk = K_WAVES * pb * K_BLOCK
    n_qk, n_pv = -(-tmax // qk_chunk), -(-tmax // pv_chunk)
    return dict(qk_bpw=qb, qk_chunk=qk_chunk, n_qk=n_qk, pv_bpw=pb, pv_chunk=pv_chunk, n_pv=n_pv,
                score_stride=max(n_qk * qk_chunk, n_pv * pv_chunk))


def qk_written_blocks(T, p):
    """Blocks whose 16 score slots q.k^T writes (every wavefront of every chunk below T)."""
    out = set()
    for c in range(p["n_qk"]):
        tok0 = c * p["qk_chunk"]
        if tok0 >= T:
            continue
        for w in range(K_WAVES):
            blk0 = tok0 // K_BLOCK + w * p["qk_bpw"]
            nb = max(0, min(p["qk_bpw"], -(-T // K_BLOCK) - blk0))
            out.update(range(blk0, blk0 + nb))
    return out


def check_sequence(T, table, num_blocks, p, sanitize=True):
    """Replays pv_kernel's indexing for one sequence; returns the number of slots checked."""
    written = qk_written_blocks(T, p)
    checked = 0
    for c in range(p["n_pv"]):
        tok0 = c * p["pv_chunk"]
        if tok0 >= T:
            continue
        for w in range(K_WAVES):
            blk0 = tok0 // K_BLOCK + w * p["pv_bpw"]
            nb = max(0, min(p["pv_bpw"], -(-T // K_BLOCK) - blk0))
            my_pb = [-1] * K_WAVE
            for lane in range(nb):
                pid = table[blk0 + lane]
                my_pb[lane] = pid if 0 <= pid < num_blocks else -1
            nst = (nb + 3) >> 2
            full_stages = min(nb, max(0, T // K_BLOCK - blk0)) >> 2
            # loads of stages 0 .. nst + 1 (two prefetched past the end), compute of 0 .. nst - 1
            for st in range(nst + 2):
                lanes = []
                for g in range(4):
                    jj = 4 * st + g
                    src = jj if jj < K_WAVE else 0
                    assert 0 <= src < K_WAVE
                    pb = my_pb[src]
                    ok = jj < nb and pb >= 0
                    blk = blk0 + jj
                    tok = min(blk, p["score_stride"] // K_BLOCK - 1) * K_BLOCK
                    assert 0 <= tok and tok + K_BLOCK <= p["score_stride"], "score load leaves the row"
                    lanes.append((ok, blk, pb))
                if st >= nst:
                    continue  # prefetched past the end: loaded, never computed
                stage_full = st < full_stages
                needs = (not stage_full) or any(not ok for ok, _, _ in lanes)
                for ok, blk, pb in lanes:
                    if needs and sanitize:
                        nvalid = min(max(T - blk * K_BLOCK, 0), K_BLOCK) if ok else 0
                    else:
                        nvalid = K_BLOCK
                    for i in range(nvalid):  # slots whose score stays finite
                        pos = blk * K_BLOCK + i
                        assert ok, f"slot of a missing block reaches the MFMA (T={T}, blk={blk})"
                        assert pos < T, f"slot past the sequence reaches the MFMA (T={T}, pos={pos})"
                        assert pb == table[blk], "page id of another block"
                        assert blk in written, f"score of block {blk} never written"
                        checked += 1
    return checked


def _table(n_blocks_needed, pool, rng, holes=0):
    ids = rng.sample(range(pool), n_blocks_needed)
    for _ in range(holes):
        ids[rng.randrange(n_blocks_needed)] = -1
    return ids


@pytest.mark.parametrize("seed", [41, 42, 43])
def test_batch32_ragged_indexing(seed):
    """The shape of test_multi_layer_batch32_ragged (28 layers, B=32, T in [2048, 32768])."""
    rng = random.Random(seed)
    lens = [rng.randint(2048, 32768) for _ in range(32)]
    p = plan(28, 32, 2, 1, 6, max(lens))
    assert p["pv_bpw"] == 64  # the shuffle's lane limit is reached
    for T in lens[:6] + [min(lens), max(lens)]:
        nblk = -(-T // K_BLOCK)
        table = _table(nblk, nblk + 500, rng)
        assert check_sequence(T, table, nblk + 500, p) == T


@pytest.mark.parametrize("T", [1, 15, 16, 17, 63, 64, 65, 1000, 4095, 4096, 4097, 18104, 32768])
@pytest.mark.parametrize("layers,B,S", [(28, 1, 1), (1, 1, 5), (28, 32, 1)])
def test_edge_lengths(T, layers, B, S):
    rng = random.Random(T * 7 + layers)
    p = plan(layers, B, 2, S, 6, max(T, 2048 if B > 1 else T))
    nblk = -(-T // K_BLOCK)
    assert check_sequence(T, _table(nblk, nblk + 64, rng), nblk + 64, p) == T


def test_invalid_block_ids_are_sanitized():
    """Holes in the block table (page id -1 or past the pool) never reach the MFMA."""
    rng = random.Random(5)
    T, pool = 5000, 1000
    nblk = -(-T // K_BLOCK)
    table = _table(nblk, pool, rng, holes=12)
    table[3] = 10**6  # past the pool
    p = plan(28, 1, 2, 1, 6, T)
    expected = sum(1 for pos in range(T) if 0 <= table[pos // K_BLOCK] < pool)
    assert expected < T
    assert check_sequence(T, table, pool, p) == expected


def test_planted_missing_sanitize_fails():
    """Without the sanitizing of partial stages, slots past T reach the MFMA."""
    rng = random.Random(9)
    T = 18104  # not a multiple of 16
    nblk = -(-T // K_BLOCK)
    p = plan(28, 32, 2, 1, 6, 32768)
    with pytest.raises(AssertionError):
        check_sequence(T, _table(nblk, nblk + 10, rng), nblk + 10, p, sanitize=False)


# ---------------------------------------------------------------------------------------------
# The `readfirstlane` question.  A build that marked pv_kernel's wavefront index wave-uniform
# (wave = readfirstlane(tid >> 6)) gave NaN in some dimensions of every query row of a head on
# four three-launch tests.  The two models below evaluate pv_compute's sanitizing inputs -- the
# stage's fullness, each lane group's nvalid, the code byte masks, the scale and score masks --
# once with the wavefront index taken per lane and once taken from the wavefront's first lane,
# and check what reaches the MFMA byte by byte.

E4M3FN_NAN = (0x7F, 0xFF)


def wave_index(tid, uniform):
    """tid >> 6 per lane, or (uniform) the first lane's value broadcast to the wavefront."""
    return ((tid - tid % K_WAVE) >> 6) if uniform else (tid >> 6)


def sanitize_masks(T, blk0, nb, my_pb, st, plant=0):
    """pv_compute's masks for stage st of one wavefront, per lane group g: (needs, [(ok, blk,
    code_keep[16], scale_keep[16], score_keep[16]) for g in 0..3]) exactly as the kernel forms
    them: code bytes through the four 32-bit words' byte masks, the scale of token n through
    n < nvalid, the BF16 scores through the 32-bit keep words (two tokens per word)."""
    full_stages = min(nb, max(0, T // K_BLOCK - blk0)) >> 2
    lanes = []
    for g in range(4):
        jj = 4 * st + g
        pb = my_pb[jj if jj < K_WAVE else 0]
        lanes.append((jj < nb and pb >= 0, blk0 + jj))
    needs = (not (st < full_stages)) or any(not ok for ok, _ in lanes)
    out = []
    for ok, blk in lanes:
        if not needs:
            out.append((ok, blk, [True] * 16, [True] * 16, [True] * 16))
            continue
        nvalid = min(max(T - blk * K_BLOCK, 0), K_BLOCK) if ok else 0
        nvalid_code = min(nvalid + plant, K_BLOCK)  # plant: a byte-mask mistake (tests only)
        code = []
        for w in range(4):
            k = min(max(nvalid_code - 4 * w, 0), 4)
            bmask = 0xFFFFFFFF if k >= 4 else (1 << (8 * k)) - 1
            code += [((bmask >> (8 * i)) & 0xFF) == 0xFF for i in range(4)]
        scale = [n < nvalid for n in range(16)]
        score = []
        for w in range(8):
            keep = 0xFFFFFFFF if 2 * w + 1 < nvalid else (0x0000FFFF if 2 * w < nvalid else 0)
            score += [(keep & 0xFFFF) == 0xFFFF, (keep >> 16) == 0xFFFF]
        out.append((ok, blk, code, scale, score))
    return needs, out


def masks_of_sequence(T, table, num_blocks, p, uniform, plant=0):
    """Every computed stage's masks for one sequence, the wavefront index taken per lane or
    wave-uniformly (the workgroup's 256 threads: tid = 64 w + lane)."""
    res = {}
    for c in range(p["n_pv"]):
        tok0 = c * p["pv_chunk"]
        if tok0 >= T:
            continue
        for tid0 in range(0, K_WAVES * K_WAVE, K_WAVE):
            waves = {wave_index(tid0 + lane, uniform) for lane in range(K_WAVE)}
            assert len(waves) == 1, "a wavefront's lanes disagree on its index"
            w = waves.pop()
            blk0 = tok0 // K_BLOCK + w * p["pv_bpw"]
            nb = max(0, min(p["pv_bpw"], -(-T // K_BLOCK) - blk0))
            my_pb = [-1] * K_WAVE
            for lane in range(nb):
                pid = table[blk0 + lane]
                my_pb[lane] = pid if 0 <= pid < num_blocks else -1
            for st in range((nb + 3) >> 2):
                res[(c, w, st)] = sanitize_masks(T, blk0, nb, my_pb, st, plant)
    return res


def _failing_shapes():
    """The three-launch shapes of the four failing tests: the B=32 ragged batch of config 4
    (lengths of test_multi_layer_batch32_ragged's seed) with tables holding holes, and short
    sequences whose last stage is partial."""
    rng = random.Random(41)
    lens = [rng.randint(2048, 32768) for _ in range(32)]
    p = plan(28, 32, 2, 1, 6, max(lens))
    cases = []
    for i, T in enumerate(lens[:8] + [17, 33, 1000, 18104]):
        nblk = -(-T // K_BLOCK)
        cases.append((T, _table(nblk, nblk + 64, rng, holes=i % 3), nblk + 64, p))
    return cases


def test_wave_uniform_index_gives_identical_sanitizing():
    """The semantically neutral change is neutral for every sanitizing input: the masks of
    every stage are the same whether the wavefront index is per lane or wave-uniform."""
    for T, table, pool, p in _failing_shapes():
        assert masks_of_sequence(T, table, pool, p, False) == masks_of_sequence(T, table, pool, p, True)


def check_masks(cases, plant=0):
    """Byte by byte: a slot that is not a token of the sequence (past T, or in a missing block
    or one with an invalid page id) reaches the MFMA with code 0, scale 0 and score -inf, and
    the stages left unsanitized hold tokens only; returns the number of non-token slots."""
    non_token_slots = 0
    for T, table, pool, p in cases:
        for (needs, lanes) in masks_of_sequence(T, table, pool, p, True, plant).values():
            for ok, blk, code, scale, score in lanes:
                for i in range(16):
                    if ok and blk * K_BLOCK + i < T:
                        assert code[i] and scale[i] and score[i], "a token of the sequence was masked"
                    else:
                        non_token_slots += 1
                        assert needs, "an unsanitized stage holds a slot that is not a token"
                        assert not code[i] and not scale[i] and not score[i], "a non-token slot keeps a value"
    return non_token_slots


def test_every_non_token_slot_is_zeroed_before_the_mfma():
    """So a NaN pattern left in an unwritten page (E4M3FN 0x7F / 0xFF) never meets p = 0 in the
    MFMA.  The failing shapes do hold such slots: with their sanitizing skipped, a NaN code byte
    among them gives NaN in its dimension for every query row, the recorded signature."""
    assert check_masks(_failing_shapes()) > 0


def test_planted_byte_mask_mistake_fails():
    """A byte mask that keeps one token too many leaks a non-token code byte."""
    with pytest.raises(AssertionError):
        check_masks(_failing_shapes(), plant=1)
