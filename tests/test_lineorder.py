"""Index arithmetic of the line-order layouts, restated and checked on the CPU.

ttsxabe_amd/csrc/lineorder.h: a 64-key reference-layout tile is staged in LDS
by load instructions that each read whole 128-byte lines, with each row's
16-byte chunks XOR-swizzled; the prefill's MFMA fragment reads then gather
from that image (pfl_kslot, pfl_vslot). ttsxabe_amd/csrc/decode.hip: the
group-1 f32 decode at head_dim 64 loads its blocks in line order too and
scatters each key's dot product over a DPP row (rs_step, fold_block_g1l,
g1l_context).

These tests restate the formulas and check what the kernels rely on: every
load lane lands in its own LDS slot and the slot holds the chunk the reads
expect; each instruction reads 8 whole lines; a fragment read's 16-lane
groups hit 16 different 16-byte bank groups (the property behind the zero
SQ_LDS_BANK_CONFLICT of the reference-layout prefill profile); and the DPP
reduce-scatter leaves every lane with the full sum of the key (or dim) the
fold assumes.
"""
import pytest


# --- lineorder.h ---------------------------------------------------------
def ksw(hd, k):
    return ((k & 3) | (((k >> 3) & 3) << 2)) if hd == 128 else (((k >> 1) & 1) | (((k >> 3) & 3) << 1))


def vsw(d):
    return (d >> 1) & 7


def kslot(hd, k, c):
    cr = hd // 8
    kpi = 64 // cr
    return (k // kpi) * 64 + (k % kpi) * cr + (c ^ ksw(hd, k))


def vslot(d, c):
    return (d >> 3) * 64 + (d & 7) * 8 + (c ^ vsw(d))


def issue_k(hd, f, lane):
    """(key, chunk) that lane `lane` of K instruction f loads (pfl_issue)."""
    cr = hd // 8
    kpi = 64 // cr
    k = f * kpi + lane // cr
    return k, (lane % cr) ^ ksw(hd, k)


def issue_v(f, lane):
    d = 8 * f + (lane >> 3)
    return d, (lane & 7) ^ vsw(d)


@pytest.mark.parametrize("hd", [64, 128])
def test_loads_fill_the_tile_with_the_chunks_the_reads_expect(hd):
    kf = hd // 8  # K instructions of a tile (and V instructions)
    seen = {}
    for f in range(kf):
        for lane in range(64):
            k, c = issue_k(hd, f, lane)
            slot = f * 64 + lane  # direct-to-LDS: lane l of instruction f
            assert kslot(hd, k, c) == slot
            seen[(k, c)] = slot
    assert len(seen) == 64 * (hd // 8) and sorted(seen.values()) == list(range(kf * 64))
    vseen = {}
    for f in range(kf):
        for lane in range(64):
            d, c = issue_v(f, lane)
            assert vslot(d, c) == f * 64 + lane
            vseen[(d, c)] = True
    assert len(vseen) == hd * 8  # every (dim, 8-key chunk) of the 64-key tile


@pytest.mark.parametrize("hd", [64, 128])
def test_each_load_instruction_reads_eight_whole_lines(hd):
    row_bytes = hd * 2  # f16 K row
    for f in range(hd // 8):
        lines = {}
        for lane in range(64):
            k, c = issue_k(hd, f, lane)
            off = k * row_bytes + 16 * c
            lines.setdefault(off // 128, set()).add(off % 128)
        assert len(lines) == 8 and all(len(v) == 8 for v in lines.values())
    for f in range(hd // 8):
        lines = {}
        for lane in range(64):
            d, c = issue_v(f, lane)
            off = d * 4096 + 16 * c  # V^T row stride: any multiple of 128 bytes
            lines.setdefault(off // 128, set()).add(off % 128)
        assert len(lines) == 8 and all(len(v) == 8 for v in lines.values())


@pytest.mark.parametrize("hd", [64, 128])
def test_fragment_reads_hit_sixteen_bank_groups(hd):
    ns, nt = hd // 32, hd // 16
    for hf in range(2):
        for t_ in range(2):
            for s in range(ns):
                for g16 in range(4):  # lanes 16*g16 .. +15 (grp = g16)
                    groups = [kslot(hd, 32 * hf + 8 * (col >> 2) + 4 * t_ + (col & 3), 4 * s + g16) % 16
                              for col in range(16)]
                    assert len(set(groups)) == 16
        for t in range(nt):
            for g16 in range(4):
                groups = [vslot(16 * t + col, 4 * hf + g16) % 16 for col in range(16)]
                assert len(set(groups)) == 16


# --- decode.hip: the group-1 f32 fold at head_dim 64 ----------------------
DPP = {
    0x140: lambda l: (l & ~15) | (15 - (l & 15)),  # row mirror
    0x141: lambda l: (l & ~7) | (7 - (l & 7)),     # half-row mirror
    0x1B: lambda l: (l & ~3) | (3 - (l & 3)),      # quad xor 3
    0xB1: lambda l: l ^ 1,                          # quad xor 1
}


def rs_step(ctrl, b, x):
    """rs_step<CTRL, B, N> over all 64 lanes: x[lane] is a list of 2N
    values (each a frozenset-tagged sum: dict term -> count)."""
    n = len(x[0]) // 2
    out = []
    for lane in range(64):
        up = (lane >> b) & 1
        src = DPP[ctrl](lane)
        sup = (src >> b) & 1
        assert sup != up  # partners keep opposite halves
        y = []
        for k in range(n):
            keep = x[lane][n + k] if up else x[lane][k]
            send = x[src][k] if sup else x[src][n + k]  # what the partner sends
            y.append(keep + send)
        out.append(y)
    return out


def test_score_reduce_scatter_gives_each_lane_its_keys_full_dot():
    # Lane l's partial dot of its instruction-i key (4i + l/16) over dims 4 (l%16) .. +3,
    # tagged as the multiset {(key, dim block)}.
    from collections import Counter
    x = [[Counter({(4 * i + (lane >> 4), lane & 15): 1}) for i in range(8)] for lane in range(64)]
    x = rs_step(0x140, 3, x)
    x = rs_step(0x141, 2, x)
    x = rs_step(0x1B, 1, x)
    for lane in range(64):
        total = x[lane][0] + x[DPP[0xB1](lane)][0]  # sc = d1 + dpp xor 1 (d1)
        key = 4 * ((lane >> 1) & 7) + (lane >> 4)  # kl in fold_block_g1l
        assert total == Counter({(key, c): 1 for c in range(16)})
    # and every key of the block is held by exactly two lanes
    keys = Counter(4 * ((lane >> 1) & 7) + (lane >> 4) for lane in range(64))
    assert sorted(keys) == list(range(32)) and set(keys.values()) == {2}


def test_context_reduce_scatter_gives_each_lane_one_dim():
    from collections import Counter
    # Lane l's context partial for dim 8i + l/8 over keys 4 (l%8) .. +3.
    x = [[Counter({(8 * i + (lane >> 3), lane & 7): 1}) for i in range(8)] for lane in range(64)]
    x = rs_step(0x141, 2, x)
    x = rs_step(0x1B, 1, x)
    x = rs_step(0xB1, 0, x)
    dims = Counter()
    for lane in range(64):
        d = 8 * (lane & 7) + (lane >> 3)  # where g1l_context's lane writes
        assert x[lane][0] == Counter({(d, kq): 1 for kq in range(8)})
        dims[d] += 1
    assert sorted(dims) == list(range(64)) and set(dims.values()) == {1}
