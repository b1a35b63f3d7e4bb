"""CPU model of the atomic schedule's split last round (the meeting protocol of
split_fixup in moe-overlap_amd/csrc/mgg_gemm.hip), run over random
interleavings of the parts.

The kernel's part q of split tile t (s = 2^L parts) meets its siblings in a
binary tree: at level l it holds the sum of the parts from b = q & -2^l, meets
the subtree b ^ 2^l on flag word s*t + (s - (s >> l)) + (q >> (l + 1)), and
either finds the sibling finished (count 1), or writes its sums to slot s*t + b
and takes a ticket (0: done; 1: winner).  The winner adds the sibling's slot and
goes on.  Checked: exactly one worker stores each tile and it holds every part
once, no slot is read before its writer finished or overwritten before it is
read, flag and slot indices stay below s * rem, and the K parts cover [0, K)
with at least two granules each.  The reference takes whole tiles
(src/triton_grouped_gemm.py:157-233); this models this build's own protocol.
"""
import random

import pytest


def run_tile(log_s, t, rng, flags, slots, stored):
    s = 1 << log_s

    def worker(q):
        held = frozenset([q])
        for lvl in range(log_s):
            fi = s * t + (s - (s >> lvl)) + (q >> (lvl + 1))
            assert s * t <= fi < s * t + s - 1
            b = q & -(1 << lvl)
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
            state, sib = slots[s * t + (b ^ (1 << lvl))]
            assert state == "ready" and not (sib & held)
            slots[s * t + (b ^ (1 << lvl))] = ("read", sib)
            held = held | sib
        stored.append((t, held))

    return [worker(q) for q in range(s)]


@pytest.mark.parametrize("log_s", [1, 2, 3])
def test_meetings_store_each_tile_once(log_s):
    s = 1 << log_s
    for seed in range(400):
        rng = random.Random(seed)
        rem = rng.randint(1, 6)
        flags, slots, stored = {}, {}, []
        gens = [g for t in range(rem) for g in run_tile(log_s, t, rng, flags, slots, stored)]
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
        assert all(v == 0 for v in flags.values())  # every winner returned its flag


@pytest.mark.parametrize("log_s", [1, 2])
def test_k_parts_cover_k(log_s):
    s = 1 << log_s
    gran = 64
    for k in range(1, 9000, 13):
        n_gran = -(-k // gran)
        if n_gran < 2 * s:
            continue
        ends = []
        for q in range(s):
            kb = ((q * n_gran) >> log_s) * gran
            ke = k if q == s - 1 else (((q + 1) * n_gran) >> log_s) * gran
            assert ke - kb > gran  # two granules, the last possibly partial
            ends.append((kb, ke))
        assert ends[0][0] == 0 and ends[-1][1] == k
        assert all(ends[i][1] == ends[i + 1][0] for i in range(s - 1))
