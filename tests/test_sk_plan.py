"""The stream-K batched decode's work partition (ttsxabe_amd/csrc/decode.hip,
attn_decode_sk_kernel), restated and checked on the CPU.

The kernel orders the batch's B (sequence, kv head, 32-key block) positions
in a flat list and prices each kv head at one cost unit for its start plus
one per block (V units in all); wave u of W = min(waves, B) takes the blocks
whose units lie in [u*V/W, (u+1)*V/W), which is empty when those units hold
only a head's start. A range
falls into segments, one per kv head: a segment that is a whole head is
written by its wave; one that is part of a head publishes a partial to the
wave's slot 0 (a segment ending before the range does) or slot 1 (the one
ending with it). The merger of a head derives the contributors owner(hs) ..
owner(he - 1) and each one's slot from the range arithmetic alone. These
tests check, over many random batches, that every partial slot is written
at most once, that each head's merger finds exactly the slots its
contributors wrote, and that every head is covered exactly once.
"""
import random

import pytest


def units(nbs, kv):
    """Per sequence: first block position, first cost unit; and the totals."""
    base, vbase, total, vtotal = [], [], 0, 0
    for nb in nbs:
        base.append(total)
        vbase.append(vtotal)
        total += nb * kv
        vtotal += (nb + 1) * kv if nb > 0 else 0
    return base, vbase, total, vtotal


def first(u, nw, plan):
    """The first block whose cost unit is at or after u*V/nw (kernel: sk_first)."""
    nbs, kv, base, vbase, total, vtotal = plan
    x = u * vtotal // nw
    if x >= vtotal:
        return total
    s = max(i for i in range(len(nbs)) if vbase[i] <= x and nbs[i] > 0)
    h, j = divmod(x - vbase[s], nbs[s] + 1)
    return base[s] + h * nbs[s] + max(j - 1, 0)


def owner(p, nw, plan):
    """The wave holding block p (kernel: sk_owner)."""
    nbs, kv, base, vbase, total, vtotal = plan
    s = max(i for i in range(len(nbs)) if base[i] <= p and nbs[i] > 0)
    off = p - base[s]
    v = vbase[s] + off + off // nbs[s] + 1
    return ((v + 1) * nw - 1) // vtotal


def simulate(nbs, kv, waves):
    base, vbase, total, vtotal = units(nbs, kv)
    if total == 0:
        return
    plan = (nbs, kv, base, vbase, total, vtotal)
    nw = min(waves, total)
    writes, contributors, whole = {}, {}, set()
    covered = []
    for u in range(nw):
        pf, pe = first(u, nw, plan), first(u + 1, nw, plan)
        assert pe >= pf
        covered += range(pf, pe)
        for pp in range(pf, pe):
            assert owner(pp, nw, plan) == u
            s = max(i for i in range(len(nbs)) if base[i] <= pp and nbs[i] > 0)
            off = pp - base[s]
            h, blk, nb = off // nbs[s], off % nbs[s], nbs[s]
            if blk == nb - 1 or pp == pe - 1:  # a segment ends here
                if blk == nb - 1 and pp - blk >= pf:
                    whole.add((s, h))
                else:
                    sl = 1 if pp == pe - 1 else 0
                    assert (u, sl) not in writes, "a slot written twice"
                    writes[(u, sl)] = (s, h)
                    contributors.setdefault((s, h), []).append(u)
    for (s, h), us in contributors.items():
        hs = base[s] + h * nbs[s]
        he = hs + nbs[s]
        c0, c1 = owner(hs, nw, plan), owner(he - 1, nw, plan)
        assert list(range(c0, c1 + 1)) == sorted(us)
        last_sl = 1 if first(c1 + 1, nw, plan) == he else 0
        for c in range(c0, c1 + 1):
            assert writes[(c, 1 if c < c1 else last_sl)] == (s, h)
        assert (s, h) not in whole
    heads = {(s, h) for s in range(len(nbs)) for h in range(kv) if nbs[s] > 0}
    assert heads == whole | set(contributors)
    assert covered == list(range(total)), "every block in exactly one range, in order"
    return plan, nw


@pytest.mark.parametrize("seed", range(6))
def test_random_batches(seed):
    rng = random.Random(seed)
    for _ in range(400):
        n = rng.randint(1, 8)
        kv = rng.choice([1, 2, 8])
        nbs = [rng.choice([0, 1, 2, 3, rng.randint(1, 300)]) for _ in range(n)]
        simulate(nbs, kv, rng.choice([1, 2, 3, 4, 8, 64, 1024]))


def test_c5_shape():
    """The C5 batch (32 sequences, 8 kv heads) over 1024 waves: a wave's
    cost (its blocks plus the kv heads starting in its range) is V / W to
    within a unit for all but a few waves (a head start on a window's last
    unit moves one unit to the next wave), and never more than two off."""
    rng = random.Random(5)
    nbs = [(rng.randint(256, 8192) + 31) // 32 for _ in range(32)]
    plan, nw = simulate(nbs, 8, 1024)
    starts = {plan[2][s] + h * nbs[s] for s in range(len(nbs)) for h in range(8)}
    cost = []
    for u in range(nw):
        pf, pe = first(u, nw, plan), first(u + 1, nw, plan)
        cost.append((pe - pf) + sum(1 for p in range(pf, pe) if p in starts))
    mean = plan[5] / nw
    assert all(abs(c - mean) < 2 for c in cost), (min(cost), max(cost), mean)
    assert sum(abs(c - mean) >= 1 for c in cost) <= nw // 100


def test_a_head_start_alone_gives_an_empty_range():
    """Units holding only a head's start give a wave no blocks; the plan
    still covers every block once and each head's contributors stay
    consecutive."""
    plan, nw = simulate([1, 300], 1, 301)
    assert first(0, nw, plan) == first(1, nw, plan)
