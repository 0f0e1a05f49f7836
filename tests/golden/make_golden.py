"""Writes tests/golden/known_answers.json: known-answer vectors for the oracle.

The reference holds no golden fixtures for the attention path (its `.golden/`
capture directory is git-ignored and absent), so these vectors are computed
here from the reference's definitions by routes that share no code with
oracle/oracle.c: Python big integers for the tests' xorshift generator
(crates/llmtie-cuda/tests/kernels.rs:35-46), exact rational/f64 arithmetic
for small attention cases, and hand-written expectations for the rounding
rules of Q8_0 (ggml roundf: half away from zero) and of the int8 twin
(crates/llmtie-cuda/src/kernels.rs:5755-5773: round half to even).

Run: python tests/golden/make_golden.py   (rewrites the JSON; deterministic)
"""
from __future__ import annotations

import json
import math
import struct
from pathlib import Path

OUT = Path(__file__).resolve().parent / "known_answers.json"
M64 = (1 << 64) - 1


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def seq_bigint(n: int, salt: int) -> list[float]:
    """kernels.rs:35-46 with explicit 64-bit wrap and the f32 operations
    `((s >> 40) as f32 / 8388608.0) * 4.0 - 2.0` done one rounding at a time
    (s >> 40 < 2^24, so the cast is exact; /2^23 and *4 are exact scalings;
    only the final subtraction rounds, and f32() applies it)."""
    s = ((salt * 0x9E3779B97F4A7C15) & M64) | 1
    out = []
    for _ in range(n):
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        out.append(f32((s >> 40) / 8388608.0 * 4.0 - 2.0))
    return out


def softmax_attend(q, ks, vs, scale):
    """Exact-as-f64 softmax attention of one query row over keys ks/values vs."""
    s = [scale * sum(a * b for a, b in zip(q, k)) for k in ks]
    m = max(s)
    e = [math.exp(x - m) for x in s]
    l = sum(e)
    hd = len(vs[0])
    return [sum(e[t] * vs[t][d] for t in range(len(ks))) / l for d in range(hd)]


def decode_hand():
    """2 query heads sharing 1 kv head, hd 2, 3 live keys of a cap-4 cache
    (the 4th slot holds a huge value that must never be read)."""
    heads, kv, hd, tk, cap, scale = 2, 1, 2, 3, 4, 0.5
    q = [1.0, 0.0, 0.0, 2.0]
    keys = [[1.0, 1.0], [2.0, -1.0], [0.0, 0.5], [1e6, 1e6]]
    vals = [[1.0, -1.0], [0.5, 2.0], [-3.0, 0.25], [1e6, 1e6]]
    k = [x for row in keys for x in row]  # [kv][cap][hd]
    v = [vals[t][d] for d in range(hd) for t in range(cap)]  # [kv][hd][cap]
    out = []
    for h in range(heads):
        out += softmax_attend(q[h * hd:(h + 1) * hd], keys[:tk], vals[:tk], scale)
    return dict(heads=heads, kv=kv, hd=hd, tk=tk, cap=cap, scale=scale, q=q, k=k, v=v, out=out)


def q8_hand():
    """One block whose amax is 127 (d = 1 exactly, id = 1): roundf sends
    every .5 away from zero. Expected codes written out by hand."""
    x = [127.0, -127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 3.49, -3.51, 0.0, 100.0] + [0.0] * 20
    codes = [127, -127, 3, -3, 1, -1, 2, -2, 3, -4, 0, 100] + [0] * 20
    return dict(x=x, codes=codes, scale_bits=0x3C00)  # f16(1.0)


def twin_hand():
    """One block with max|y| = 127: d = 127 * f32(1/127) = 1 exactly (checked
    below), inv = 1, and rint sends .5 to the even neighbour. A second block
    of zeros gets scale 0 and codes 0."""
    r = f32(1.0 / 127.0)
    assert f32(127.0 * r) == 1.0
    y = [127.0, -127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 3.5, -3.5, 0.49, 126.5] + [0.0] * 20
    codes = [127, -127, 2, -2, 0, 0, 2, -2, 4, -4, 0, 126] + [0] * 20
    return dict(y=y + [0.0] * 32, codes=codes + [0] * 32, scales=[1.0, 0.0])


def main():
    g = {
        "seq": {str(salt): seq_bigint(48, salt) for salt in (1, 71, 72, 73, 300, 301, 302)},
        "decode_hand": decode_hand(),
        "q8_hand": q8_hand(),
        "twin_hand": twin_hand(),
    }
    OUT.write_text(json.dumps(g, indent=1) + "\n")
    print("wrote", OUT)


if __name__ == "__main__":
    main()
