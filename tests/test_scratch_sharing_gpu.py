"""One decode scratch shared by calls of every kind and shape.

Split partials and arrival counters live in the scratch between calls: a
call that left a counter off zero, or a merge that read a partial another
call of another shape had written, would give a result that differs from
the same call on a fresh scratch. Each call here is compared bit for bit
with that.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.test_q8_decode_gpu import load, random_q8_cache
from tests.util import down, up, up_f16

pytestmark = pytest.mark.gpu


def test_every_decode_kind_through_one_scratch(gpu):
    from ttsxabe_amd.gpu import DecodeScratch, KvCacheQ8

    calls = []

    def f16_case(heads, kv, hd, tk, cap, salt):
        q = up(oracle.seq(heads * hd, salt))
        k = up_f16(oracle.seq(kv * cap * hd, salt + 1))
        v = up_f16(oracle.seq(kv * hd * cap, salt + 2))
        return lambda s: down(gpu.attn_decode_f16(q, k, v, heads, kv, hd, tk, cap, 0.11, False, s))

    def f32_case(heads, kv, hd, tk, cap, salt):
        q = up(oracle.seq(heads * hd, salt))
        k = up(oracle.seq(kv * cap * hd, salt + 1))
        v = up(oracle.seq(kv * hd * cap, salt + 2))
        return lambda s: down(gpu.attn_decode(q, k, v, heads, kv, hd, tk, cap, 0.125, True, s))

    def q8_case(hd, heads, kv, slots, cap, tk, seed):
        cache = KvCacheQ8(slots, kv, hd, cap)
        load(cache, *random_q8_cache(slots, kv, hd, cap, seed))
        nseq = len(tk)
        q = up(oracle.normal(nseq * heads * hd, seed + 7))
        tkd = up(np.asarray(tk, np.int32), torch.int32)
        sld = up(np.arange(nseq, dtype=np.int32) % slots, torch.int32)
        return lambda s: down(gpu.attn_decode_q8_batch(q, cache, tkd, sld, int(max(tk)), heads, hd ** -0.5, False, s))

    calls.append(("f16 32/8/128 tk 4096 (one XCD per head)", f16_case(32, 8, 128, 4096, 4096, 900)))
    calls.append(("q8 batch of 5 (stream-K)", q8_case(128, 32, 8, 5, 2048, [2000, 31, 1500, 700, 2048], 901)))
    calls.append(("f16 4/2/128 tk 16500 (two-phase merge)", f16_case(4, 2, 128, 16500, 16512, 902)))
    calls.append(("f32 8/8/64 tk 5000", f32_case(8, 8, 64, 5000, 5056, 903)))
    calls.append(("q8 batch of 70 (planned grid)", q8_case(128, 8, 2, 70, 320, list(range(5, 285, 4)), 904)))
    calls.append(("f16 40/40/128 tk 1500", f16_case(40, 40, 128, 1500, 1536, 905)))

    fresh = [fn(DecodeScratch()) for _, fn in calls]
    shared = DecodeScratch()
    for rep in range(3):
        for (name, fn), want in zip(calls, fresh):
            got = fn(shared)
            assert np.array_equal(got, want, equal_nan=True), f"{name}, pass {rep}"
