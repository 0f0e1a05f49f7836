"""The stream-K batched decode's work partition (ttsxabe_amd/csrc/decode.hip,
attn_decode_sk_kernel), restated and checked on the CPU.

The kernel gives wave u of W the flat range [u*B/W, (u+1)*B/W) of the batch's
B (sequence, kv head, 32-key block) positions, W = min(waves, B). A range
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


def first(u, nw, total):
    return u * total // nw


def owner(p, nw, total):
    return ((p + 1) * nw - 1) // total


def simulate(nbs, kv, waves):
    base, total = [], 0
    for nb in nbs:
        base.append(total)
        total += nb * kv
    if total == 0:
        return
    nw = min(waves, total)
    writes, contributors, whole = {}, {}, set()
    for u in range(nw):
        pf, pe = first(u, nw, total), first(u + 1, nw, total)
        assert pe > pf, "every wave's range is non-empty"
        for pp in range(pf, pe):
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
        c0, c1 = owner(hs, nw, total), owner(he - 1, nw, total)
        assert list(range(c0, c1 + 1)) == sorted(us)
        last_sl = 1 if first(c1 + 1, nw, total) == he else 0
        for c in range(c0, c1 + 1):
            assert writes[(c, 1 if c < c1 else last_sl)] == (s, h)
        assert (s, h) not in whole
    heads = {(s, h) for s in range(len(nbs)) for h in range(kv) if nbs[s] > 0}
    assert heads == whole | set(contributors)


@pytest.mark.parametrize("seed", range(6))
def test_random_batches(seed):
    rng = random.Random(seed)
    for _ in range(400):
        n = rng.randint(1, 8)
        kv = rng.choice([1, 2, 8])
        nbs = [rng.choice([0, 1, 2, 3, rng.randint(1, 300)]) for _ in range(n)]
        simulate(nbs, kv, rng.choice([1, 2, 3, 4, 8, 64, 1024]))


def test_c5_shape():
    """The C5 batch (32 sequences, 8 kv heads) over 1024 waves."""
    rng = random.Random(5)
    nbs = [(rng.randint(256, 8192) + 31) // 32 for _ in range(32)]
    simulate(nbs, 8, 1024)
