"""CPU model of the persistent kernel's work distribution with the
device-derived queue (run_worker and decode in
moe-overlap_amd/csrc/mgg_gemm_kernel.h): the grouped tile order inside an
expert and the atomic schedule's static rounds followed by tickets.

Checked over many shapes and random finishing orders: the grouped order maps
an expert's item indices onto its (tile_m, tile_n) tiles one to one; every
work item is taken exactly once; the worker that draws the last ticket is the
last to draw one (it hands the counter word on), and W + G tickets are drawn
in all, the value the reference's counter ends at
(src/triton_grouped_gemm.py:157-233, each worker over-fetches once).  The
reference deals every item after the first round by ticket; the static rounds
and the grouped order are this build's placement, which these invariants keep
equivalent.
"""
import random

import pytest


def grouped_tile(local, mt_e, n_tiles, group_m=4):
    """(tm, tn) of item `local` of an expert with mt_e m-tiles: groups of
    group_m m-tiles, each taken n-tile by n-tile."""
    span = group_m * n_tiles
    g = local // span
    gm = min(group_m, mt_e - g * group_m)
    sub = local - g * span
    tn = sub // gm
    return g * group_m + (sub - tn * gm), tn


@pytest.mark.parametrize("group_m", [1, 2, 4])
def test_grouped_order_is_a_bijection(group_m):
    for mt_e in range(1, 14):
        for n_tiles in range(1, 41):
            tiles = [grouped_tile(i, mt_e, n_tiles, group_m) for i in range(mt_e * n_tiles)]
            assert sorted(tiles) == [(m, n) for m in range(mt_e) for n in range(n_tiles)]


def test_grouped_order_keeps_an_xcd_share_compact():
    # 32 n-tiles (N = 8192 at 256 columns): 32 consecutive items span 4 m-tiles x 8 n-tiles.
    for start in range(0, 4 * 32, 32):
        share = [grouped_tile(i, 4, 32) for i in range(start, start + 32)]
        assert len({m for m, _ in share}) == 4 and len({n for _, n in share}) == 8


def simulate(w_tiles, g, split_s, rng, atomic=True):
    """Workers 0..g-1 (first item = worker index); items below dyn_base go by
    stripes (item + g), later ones by tickets t -> dyn_base + t in the order
    workers finish (random).  Returns the items taken and the ticket log."""
    rem = w_tiles % g if w_tiles > g else w_tiles
    w_base = w_tiles - rem if split_s > 1 else w_tiles
    w = w_base + rem * split_s if split_s > 1 else w_tiles
    dyn_base = (w_tiles // g) * g if (atomic and w_tiles >= 2 * g) else g
    last_ticket = w - dyn_base + g - 1 if w > g else w - 1
    taken, tickets = [], []
    # each active worker: its current item; event loop picks a random worker to finish
    active = {v: v for v in range(min(g, w))}
    counter = 0
    while active:
        v = rng.choice(sorted(active))
        item = active[v]
        taken.append(item)
        if item + g >= dyn_base:  # next by ticket
            t = counter
            counter += 1
            tickets.append(t)
            nxt = dyn_base + t
        else:
            nxt = item + g
        if nxt < w:
            active[v] = nxt
        else:
            del active[v]
    return sorted(taken), tickets, w, last_ticket


@pytest.mark.parametrize("seed", range(4))
def test_static_rounds_then_tickets_take_every_item_once(seed):
    rng = random.Random(seed)
    for _ in range(300):
        g = rng.choice([2, 3, 5, 8, 12, 64, 256])
        w_tiles = rng.randint(1, 6 * g)
        rem = w_tiles % g if w_tiles > g else w_tiles
        split_s = 1
        for sp in (4, 3, 2):
            if rem > 0 and rem * sp <= g and rng.random() < 0.7:
                split_s = sp
                break
        taken, tickets, w, last_ticket = simulate(w_tiles, g, split_s, rng)
        assert taken == list(range(w))
        dyn_base = w_tiles // g * g if w_tiles >= 2 * g else g
        # one ticket per item past the stripes, plus each worker's one past the queue
        assert len(tickets) == (w - dyn_base + g if w > g else w)
        assert tickets[-1] == last_ticket == len(tickets) - 1
        if split_s == 1 and w_tiles > g:
            # the stripes stand for the first dyn_base tickets: W + G in all, as in the reference
            assert dyn_base + len(tickets) == w_tiles + g
