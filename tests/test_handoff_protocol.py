"""CPU model of the decode kernel's split-K hand-off (kivi_decode_mfma.hip:
stream_run's partial stores and flags, merge_segments' polling merge), run
under random interleavings of every wavefront's memory operations.

What the kernel does, restated as the model's rules:
- the stream of units is cut into W runs by the weighted split (run_begin /
  wave_of: the first nw runs -- the fused step's writer wavefronts -- weigh
  kWriterRun / kRun of the others); a run that covers only part of a segment
  stores its piece's partial in slot seg + w, and after its run waits for all
  its stores (vmcnt(0)) and then stores the launch's epoch in that slot's
  flag;
- a merge workgroup recomputes the segment's pieces from the same split; with
  more than one non-empty piece it waits for the first pending piece's flag,
  takes the prefix of pieces whose flags show the epoch, loads their
  partials, clears those flags and folds them in piece order;
- a replayed HIP graph repeats its launch's epoch; the workspace keeps its
  contents between launches.

The checks: every cut segment is merged exactly once from exactly its pieces,
in piece order, with the values of the launch that merges it -- under random
schedules, across back-to-back replays with one epoch -- and two mutants of
the protocol (no flag clear, flag before the data is complete) are caught.
"""
from __future__ import annotations

import random

import pytest

K_RUN, K_WRITER_RUN = 16, 13  # kivi_decode_mfma.hip: kRun, kWriterRun


def weight_sum(w: int, nw: int) -> int:
    return K_RUN * w - (K_RUN - K_WRITER_RUN) * min(w, nw)


def run_begin(w: int, tt: int, W: int, nw: int) -> int:
    return tt * weight_sum(w, nw) // weight_sum(W, nw)


def wave_of(x: int, tt: int, W: int, nw: int) -> int:
    c = x * weight_sum(W, nw) // tt
    n = min(nw, W)
    w = c // K_WRITER_RUN if c < K_WRITER_RUN * n else n + (c - K_WRITER_RUN * n) // K_RUN
    w = min(w, W - 1)
    while w > 0 and run_begin(w, tt, W, nw) > x:
        w -= 1
    while w + 1 < W and run_begin(w + 1, tt, W, nw) <= x:
        w += 1
    return w


def test_weighted_split_inverts():
    """wave_of is the inverse of run_begin for every unit, with and without
    writer runs, at the kernel's run counts (W at most a quarter of the units)."""
    rng = random.Random(1)
    for _ in range(400):
        tt = rng.randint(1, 300000)
        W = min(rng.randint(1, 3072), max(1, (tt + 3) // 4))
        nw = rng.choice([0, 1, 7, 128, W, W + 5])
        bounds = [run_begin(w, tt, W, nw) for w in range(W + 1)]
        assert bounds[0] == 0 and bounds[-1] == tt
        assert all(a <= b for a, b in zip(bounds, bounds[1:]))
        for _ in range(30):
            x = rng.randrange(tt)
            w = wave_of(x, tt, W, nw)
            assert bounds[w] <= x < bounds[w + 1]
        if 0 < nw < W and tt >= 64 * W:  # writer runs are shorter than the others
            assert bounds[1] - bounds[0] < bounds[W] - bounds[W - 1]


class Memory:
    """Stores become visible in any order until the issuing wave waits for
    them (vmcnt(0)); loads read what is visible."""

    def __init__(self):
        self.cells: dict = {}

    def load(self, key, default=None):
        return self.cells.get(key, default)


def launch(mem: Memory, segs: list[int], W: int, nw: int, epoch: int, tag: int,
           rng: random.Random, merge_wgs: int, *, clear_flags=True, wait_before_flag=True):
    """One decode launch under a random schedule.  Returns {seg: folded
    pieces} for merged segments and {seg: piece} for whole ones."""
    tt = sum(segs)
    starts = [sum(segs[:i]) for i in range(len(segs))]
    out: dict = {}

    def pieces_of(seg):
        s0, s1 = starts[seg], starts[seg] + segs[seg]
        w0, w1 = wave_of(s0, tt, W, nw), wave_of(s1 - 1, tt, W, nw)
        res = []
        for w in range(w0, w1 + 1):
            a, b = max(run_begin(w, tt, W, nw), s0), min(run_begin(w + 1, tt, W, nw), s1)
            if a < b:
                res.append((w, a, b))
        return res

    def stream_wave(w):
        x0, x1 = run_begin(w, tt, W, nw), run_begin(w + 1, tt, W, nw)
        pending = []  # stores not yet visible
        cut = []
        for seg in range(len(segs)):
            s0, s1 = starts[seg], starts[seg] + segs[seg]
            a, b = max(x0, s0), min(x1, s1)
            if a >= b:
                continue
            yield
            value = (tag, seg, a, b)  # the partial this launch computes
            if (a, b) == (s0, s1):
                out[seg] = value
            else:
                pending.append((("part", seg + w), value))
                cut.append(seg + w)
        while pending:  # the stores land in any order, interleaved with others
            if not wait_before_flag and cut:
                break
            i = rng.randrange(len(pending))
            k, v = pending.pop(i)
            mem.cells[k] = v
            yield
        for slot in cut:
            mem.cells[("flag", slot)] = epoch
            yield
        while pending:  # the mutant's late data
            k, v = pending.pop()
            mem.cells[k] = v
            yield

    def merge_wave(m):
        for seg in range(m, len(segs), merge_wgs):
            ps = pieces_of(seg)
            if len(ps) <= 1:
                continue
            todo = list(ps)
            folded = []
            while todo:
                while mem.load(("flag", seg + todo[0][0])) != epoch:
                    yield  # the one-lane wait
                ready = []
                for p in todo:  # the ballot round: the landed prefix
                    if mem.load(("flag", seg + p[0])) != epoch:
                        break
                    ready.append(p)
                yield
                for p in ready:
                    folded.append(mem.load(("part", seg + p[0])))
                    if clear_flags:
                        mem.cells[("flag", seg + p[0])] = 0
                todo = todo[len(ready):]
                yield
            out[seg] = tuple(folded)

    agents = [stream_wave(w) for w in range(W)] + [merge_wave(m) for m in range(merge_wgs)]
    live = list(agents)
    steps = 0
    while live:
        a = rng.choice(live)
        try:
            next(a)
        except StopIteration:
            live.remove(a)
        steps += 1
        assert steps < 10_000_000, "schedule did not drain"
    expected = {}
    for seg in range(len(segs)):
        ps = pieces_of(seg)
        if len(ps) == 1:
            expected[seg] = (tag, seg, ps[0][1], ps[0][2])
        else:
            expected[seg] = tuple((tag, seg, a, b) for _, a, b in ps)
    return out, expected


def random_case(rng):
    nseg = rng.randint(1, 12)
    segs = [rng.randint(1, 40) for _ in range(nseg)]
    tt = sum(segs)
    W = rng.randint(1, max(1, min(24, tt // 2)))
    nw = rng.choice([0, 0, 1, 3, W])
    merge_wgs = rng.randint(1, max(1, min(nseg, W)))
    return segs, W, nw, merge_wgs


def test_every_cut_segment_merged_once_from_its_pieces():
    """Random segment lengths, run counts, writer runs and schedules: every
    segment's output is its whole piece, or the fold of exactly its pieces in
    piece order, with this launch's values."""
    rng = random.Random(7)
    for _ in range(300):
        segs, W, nw, mw = random_case(rng)
        out, expected = launch(Memory(), segs, W, nw, epoch=0xABC, tag=1, rng=rng, merge_wgs=mw)
        assert out == expected


def test_graph_replays_read_no_stale_partials():
    """Back-to-back launches with one epoch on one workspace (a replayed
    graph): each launch merges its own partials only."""
    rng = random.Random(11)
    for _ in range(150):
        segs, W, nw, mw = random_case(rng)
        mem = Memory()
        for rep in range(4):
            out, expected = launch(mem, segs, W, nw, epoch=0xE0, tag=rep, rng=rng, merge_wgs=mw)
            assert out == expected, f"replay {rep}"


@pytest.mark.parametrize("mutant", ["no_clear", "flag_first"])
def test_protocol_mutants_are_caught(mutant):
    """Without the flag clear a replay's merge folds the previous replay's
    partials; with the flag stored before the data is complete a merge reads
    stale data.  Some schedule shows each."""
    rng = random.Random(13)
    kw = {"clear_flags": mutant != "no_clear", "wait_before_flag": mutant != "flag_first"}
    caught = False
    for _ in range(400):
        segs, W, nw, mw = random_case(rng)
        mem = Memory()
        for rep in range(3):
            out, expected = launch(mem, segs, W, nw, epoch=0xE0, tag=rep, rng=rng,
                                   merge_wgs=mw, **kw)
            if out != expected:
                caught = True
                break
        if caught:
            break
    assert caught
