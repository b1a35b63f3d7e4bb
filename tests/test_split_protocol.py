"""CPU model of the atomic schedule's split last round (the meeting protocol of
split_fixup in moe-overlap_amd/csrc/mgg_gemm_kernel.h), run over random
interleavings of the parts.

The kernel's part q of split tile t (s parts, any s >= 2) meets its siblings in
a binary tree: at level l it holds the sum of the parts from b = q & -2^l, and
when the sibling subtree b ^ 2^l exists (< s) it meets that subtree's holder on
flag word (s-1)*t + (pairs of the levels below l) + (q >> (l + 1)), and either
finds the sibling finished (count 1), or writes its sums to slot s*t + b and
takes a ticket (0: done; 1: winner).  The winner adds the sibling's slot and
goes on.  Checked: exactly one worker stores each tile and it holds every part
once, no slot is read before its writer finished or overwritten before it is
read, flag indices stay inside the tile's s - 1 words and slot indices inside
its s, and the K parts (cut unevenly) cover [0, K).  The
reference takes whole tiles (src/triton_grouped_gemm.py:157-233); this models
this build's own protocol.
"""
import random

import pytest


def run_tile(s, t, rng, flags, slots, stored):
    def worker(q):
        held = frozenset([q])
        level_flags, subtrees, lvl = (s - 1) * t, s, 0
        while (1 << lvl) < s:
            b = q & -(1 << lvl)
            fi = level_flags + (q >> (lvl + 1))
            level_flags += subtrees >> 1
            subtrees = (subtrees + 1) >> 1
            sib = b ^ (1 << lvl)
            lvl += 1
            if sib >= s:
                continue
            assert (s - 1) * t <= fi < (s - 1) * (t + 1)
            yield
            last = flags.get(fi, 0) == 1  # peek
            if not last:
                slots[s * t + b] = ("ready", held)
                yield
                count = flags.get(fi, 0)
                flags[fi] = count + 1  # ticket
                last = count == 1
            if not last:
                return
            flags[fi] = 0
            yield
            state, sibling = slots[s * t + sib]
            assert state == "ready" and not (sibling & held)
            slots[s * t + sib] = ("read", sibling)
            held = held | sibling
        stored.append((t, held))

    return [worker(q) for q in range(s)]


@pytest.mark.parametrize("s", [2, 3, 4, 5, 6, 7, 8])
def test_meetings_store_each_tile_once(s):
    for seed in range(300):
        rng = random.Random(seed)
        rem = rng.randint(1, 6)
        flags, slots, stored = {}, {}, []
        gens = [g for t in range(rem) for g in run_tile(s, t, rng, flags, slots, stored)]
        alive = list(range(len(gens)))
        while alive:
            i = rng.choice(alive)
            try:
                next(gens[i])
            except StopIteration:
                alive.remove(i)
        assert sorted(t for t, _ in stored) == list(range(rem))
        assert all(held == frozenset(range(s)) for _, held in stored)
        assert all(0 <= k < s * rem for k in slots)
        assert all(0 <= k < (s - 1) * rem for k in flags)
        assert all(v == 0 for v in flags.values())  # every winner returned its flag


@pytest.mark.parametrize("s", [2, 3, 4])
@pytest.mark.parametrize("gran", [32, 64, 128])
def test_k_parts_cover_k(s, gran):
    """Parts are taken only when an even cut would give each at least 1024 of
    K (as many granules as that takes); they then tile [0, K), and part q is
    d granules (384 of K, rounded up) shorter per bit set in q than part 0,
    to within a granule of rounding (the last part's last granule possibly
    partial), every part keeping more than a quarter of 1024."""
    min_gran = -(-1024 // gran)
    d = -(-384 // gran)

    def pc_sum(p):
        return sum(bin(j).count("1") for j in range(1, p))

    def bound(p, n_gran):
        return p * (n_gran + d * pc_sum(s)) // s - d * pc_sum(p)

    for k in range(1, 20000, 13):
        n_gran = -(-k // gran)
        if n_gran < min_gran * s:
            continue
        ends = []
        for q in range(s):
            kb = 0 if q == 0 else bound(q, n_gran) * gran
            ke = k if q == s - 1 else bound(q + 1, n_gran) * gran
            assert ke - kb > 256
            ends.append((kb, ke))
        g0 = ends[0][1] - ends[0][0]
        for q in range(1, s):
            gq = ends[q][1] - ends[q][0]
            want = g0 - d * gran * bin(q).count("1")
            assert abs(gq - want) <= 2 * gran, (k, q, gq, want)
        assert ends[0][0] == 0 and ends[-1][1] == k
        assert all(ends[i][1] == ends[i + 1][0] for i in range(s - 1))
