"""The bookkeeping of decode attention split by work (k_attn_stream and
k_attn_stream_merge in qubivex_amd/csrc/kernels.hip), restated on the CPU: workgroup w
takes the slots [floor(w T / P), floor((w + 1) T / P)) of the unit-major work order, where
each unit holds `cost` set-up slots (its per-unit overhead, no tiles) and then one slot per
tile; a unit whose tiles lie wholly inside one range is written out directly, a unit cut
by range boundaries leaves one partial per workgroup whose range holds some of its tiles,
in slot 0 (the workgroup's first unit with tiles) or 1 (its last); the merge finds them
from the unit's range alone.  Every unit's
tiles must be covered exactly once and the merge must read exactly the slots that were
written (a partial read from a workgroup with an empty range would be garbage)."""
import random

import pytest


def split(tiles, upi, P, cost=0):
    cum = [0]
    for t in tiles:
        cum.append(cum[-1] + (t + cost) * upi)
    T = cum[-1]
    written = {}
    for w in range(P):
        s0, s1 = w * T // P, (w + 1) * T // P
        x, first = s0, True
        while x < s1:
            item = max(i for i in range(len(tiles)) if cum[i] <= x and cum[i + 1] > x)
            per = (cum[item + 1] - cum[item]) // upi
            rel = x - cum[item]
            ul = rel // per
            tiles_at = cum[item] + ul * per + cost
            uend = cum[item] + (ul + 1) * per
            seg = min(uend, s1)
            if seg <= tiles_at:  # set-up slots only
                x = seg
                continue
            t0, t1 = max(x - tiles_at, 0), seg - tiles_at
            full = t0 == 0 and seg == uend
            written.setdefault((item, ul), []).append(
                ("out", None, t0, t1) if full else ("part", 2 * w + (0 if first else 1), t0, t1))
            first, x = False, seg
    return cum, T, written


def merge_reads(cum, T, P, item, ul, upi, cost=0):
    per = (cum[item + 1] - cum[item]) // upi
    a0 = cum[item] + ul * per
    a, b = a0 + cost, a0 + per
    owner = lambda x: ((x + 1) * P + T - 1) // T - 1  # noqa: E731
    w0, w1 = owner(a), owner(b - 1)
    if w0 == w1:
        return None
    start0 = w0 * T // P
    return {2 * w + (1 if (w == w0 and start0 < a0) else 0)
            for w in range(w0, w1 + 1) if w * T // P != (w + 1) * T // P}


@pytest.mark.parametrize("cost", [0, 1, 6, 40])
@pytest.mark.parametrize("seed", range(6))
def test_every_tile_once_and_the_merge_reads_what_was_written(seed, cost):
    r = random.Random(seed * 100 + cost)
    for _ in range(60):
        tiles = [r.randint(1, 300) for _ in range(r.randint(1, 30))]
        upi = r.choice([1, 2, 4, 8, 16])
        P = r.choice([1, 2, 7, 64, 396, 1536, sum(tiles) * upi + 5])
        cum, T, written = split(tiles, upi, P, cost)
        for item in range(len(tiles)):
            for ul in range(upi):
                got = written[(item, ul)]
                cover = sorted((t0, t1) for _, _, t0, t1 in got)
                assert cover[0][0] == 0 and cover[-1][1] == tiles[item]
                assert all(cover[i][1] == cover[i + 1][0] for i in range(len(cover) - 1))
                reads = merge_reads(cum, T, P, item, ul, upi, cost)
                if reads is None:
                    assert [k for k, *_ in got] == ["out"]
                else:
                    assert all(k == "part" for k, *_ in got)
                    assert reads == {s for _, s, _, _ in got}


def test_the_check_catches_reads_from_empty_workgroups():
    """Positive control: the merge without the empty-range rule reads slots nobody wrote
    when there are more workgroups than tiles (9 items of 1..44 tiles, 396 workgroups)."""
    tiles = [(n + 15) // 16 for n in [1, 15, 17, 33, 47, 48, 49, 149, 700]]
    upi, P = 4, 396
    cum, T, written = split(tiles, upi, P)
    wrong = 0
    for item in range(len(tiles)):
        for ul in range(upi):
            per = (cum[item + 1] - cum[item]) // upi
            a = cum[item] + ul * per
            owner = lambda x: ((x + 1) * P + T - 1) // T - 1  # noqa: E731
            w0, w1 = owner(a), owner(a + per - 1)
            if w0 == w1:
                continue
            start0 = w0 * T // P
            unfiltered = {2 * w + (1 if (w == w0 and a != start0) else 0) for w in range(w0, w1 + 1)}
            wrong += unfiltered != {s for _, s, _, _ in written[(item, ul)]}
    assert wrong > 0


def test_the_check_catches_a_slot_rule_that_ignores_set_up_slots():
    """Positive control: with set-up slots, taking slot 1 for w0 whenever the unit's first
    tile is not w0's first slot (the rule without set-up slots) reads a slot nobody wrote
    when w0's range starts inside the unit's set-up slots."""
    r = random.Random(7)
    wrong = 0
    for _ in range(40):
        tiles = [r.randint(1, 60) for _ in range(r.randint(2, 12))]
        upi, P, cost = r.choice([1, 4, 8]), r.choice([7, 64, 396]), 6
        cum, T, written = split(tiles, upi, P, cost)
        owner = lambda x: ((x + 1) * P + T - 1) // T - 1  # noqa: E731
        for item in range(len(tiles)):
            for ul in range(upi):
                per = (cum[item + 1] - cum[item]) // upi
                a = cum[item] + ul * per + cost
                w0, w1 = owner(a), owner(cum[item] + (ul + 1) * per - 1)
                if w0 == w1:
                    continue
                old = {2 * w + (1 if (w == w0 and a != w0 * T // P) else 0)
                       for w in range(w0, w1 + 1) if w * T // P != (w + 1) * T // P}
                wrong += old != {s for _, s, _, _ in written[(item, ul)]}
    assert wrong > 0
