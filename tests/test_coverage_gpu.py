"""Paths the reference's own test shapes do not reach.

- Decode with the widest GQA groups the kernel takes (8 and 16 query heads
  per kv head), and the single-split short-context plan.
- The batched Q8_0 decode at the edges of its device-side plan: one
  sequence, 64 sequences (the largest device-planned batch), 65 (the
  host-planned grid), and one-position sequences.
- The prefill's staged fallback for a non-positive score scale.
- The f32-cache prefill (staged through registers inside the kernel): two
  streams at once, and a first use inside a captured graph.
Bars as elsewhere: decode 2e-5 of full scale against the exact f64 value;
Q8_0 1e-3 (one f16 rounding of P * d_v); prefill the reference's rule.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.test_q8_decode_gpu import dequant_seq, load, random_q8_cache
from tests.util import down, full_scale_err, up, up_f16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("heads,kv,hd,tk,cap", [(32, 2, 128, 3000, 3072), (16, 1, 64, 500, 512), (64, 8, 128, 96, 128)])
def test_wide_groups_and_short_contexts(gpu, heads, kv, hd, tk, cap):
    from ttsxabe_amd.gpu import DecodeScratch, TiledCache16
    q = oracle.seq(heads * hd, 41)
    k0 = oracle.seq(kv * cap * hd, 42)
    v0 = oracle.seq(kv * hd * cap, 43)
    k, v = oracle.through_f16(k0), oracle.through_f16(v0)
    exact = oracle.decode_f64(q, k, v, heads, kv, hd, tk, cap, 0.09, False)
    s = DecodeScratch()
    dk, dv = up_f16(k0), up_f16(v0)
    a = down(gpu.attn_decode_f16(up(q), dk, dv, heads, kv, hd, tk, cap, 0.09, False, s))
    assert full_scale_err(exact, a) < 2e-5
    t = TiledCache16(kv, hd, cap)
    gpu.t16_from_ref(dk, dv, t, tk)
    assert np.array_equal(a, down(gpu.attn_decode_t16(up(q), t, heads, tk, 0.09, False, s)))


@pytest.mark.parametrize("nseq", [1, 64, 65])
def test_q8_batch_at_the_edges_of_its_plan(gpu, nseq):
    from ttsxabe_amd.gpu import DecodeScratch, KvCacheQ8
    hd, heads, kv, slots, cap = 128, 8, 2, 7, 512
    kc, ks, vc, vs = random_q8_cache(slots, kv, hd, cap, 61)
    cache = KvCacheQ8(slots, kv, hd, cap)
    load(cache, kc, ks, vc, vs)
    rng = np.random.default_rng(nseq)
    tk = rng.integers(1, cap + 1, nseq).astype(np.int32)
    tk[::5] = 1                       # one-position sequences
    slot = rng.integers(0, slots, nseq).astype(np.int32)
    q = oracle.normal(nseq * heads * hd, 62)
    got = down(gpu.attn_decode_q8_batch(up(q), cache, up(tk, torch.int32), up(slot, torch.int32), cap, heads,
                                        0.088, False, DecodeScratch()))
    n = heads * hd
    for i in range(nseq):
        k, v = dequant_seq(kc, ks, vc, vs, slot[i], kv, hd, cap)
        exact = oracle.decode_f64(q[i * n:(i + 1) * n], k, v, heads, kv, hd, int(tk[i]), cap, 0.088, False)
        assert full_scale_err(exact, got[i * n:(i + 1) * n]) < 1e-3, f"seq {i} tk {tk[i]}"


@pytest.mark.parametrize("scale", [-0.125, 0.0])
def test_prefill_with_a_non_positive_scale_takes_the_staged_path(gpu, scale):
    tq, heads, kv, hd, cap = 40, 4, 2, 128, 64
    q = oracle.seq(tq * heads * hd, 51) - 2.0
    k = oracle.seq(kv * cap * hd, 52)
    v = oracle.seq(kv * hd * cap, 53)
    want, spread = oracle.prefill_ref(q, heads * hd, k, v, tq, 0, heads, kv, hd, cap, scale, True)
    got = down(gpu.flash_attn_f16(up(q), up_f16(k), up_f16(v), tq, 0, heads, kv, hd, cap, scale, True))
    tol = 2e-4 + 1e-2 * np.abs(want) + 1e-2 * spread
    assert (np.abs(got - want) / tol).max() < 0.5


def test_f32_prefill_on_two_streams_at_once(gpu):
    # Two f32-cache prefills in flight on two streams share no state.
    hd, heads, kv = 128, 8, 2
    cases = []
    for tq, salt in ((300, 1), (700, 2)):
        cap = tq
        q = oracle.seq(tq * heads * hd, salt) - 2.0
        k = oracle.seq(kv * cap * hd, salt + 10)
        v = oracle.seq(kv * hd * cap, salt + 20)
        cases.append((tq, cap, up(q), up(k), up(v)))
    ref = [down(gpu.flash_attn(q, k, v, tq, 0, heads, kv, hd, cap, 0.088, True)) for tq, cap, q, k, v in cases]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [None, None]
    for rep in range(3):
        for i, (s, (tq, cap, q, k, v)) in enumerate(zip(streams, cases)):
            with torch.cuda.stream(s):
                outs[i] = gpu.flash_attn(q, k, v, tq, 0, heads, kv, hd, cap, 0.088, True)
        torch.cuda.synchronize()
        for i in range(2):
            assert np.array_equal(down(outs[i]), ref[i]), f"stream {i} rep {rep}"


def test_f32_prefill_first_used_inside_a_graph(gpu):
    # The f32 cache is staged inside the kernel (nothing is allocated), so a
    # first call made under capture is an ordinary kernel node: every replay
    # must equal the eager result.
    hd, heads, kv, tq = 64, 4, 4, 1000
    q = up(oracle.seq(tq * heads * hd, 71) - 2.0)
    k = up(oracle.seq(kv * tq * hd, 72))
    v = up(oracle.seq(kv * hd * tq, 73))
    eager = down(gpu.flash_attn(q, k, v, tq, 0, heads, kv, hd, tq, 0.125, False))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            out = gpu.flash_attn(q, k, v, tq, 0, heads, kv, hd, tq, 0.125, False)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(down(out), eager), f"replay {rep}"
