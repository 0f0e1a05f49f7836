"""HIP-graph capture of the path, as bench.py times it: every replay, with
the program's own eager work and synchronisations between replays, must give
the eager result bit for bit. Covers the decode's split hand-off (arrival
counters left at zero by every call, so a replay starts clean), the two-phase
merge, the batched Q8_0 decode, the prefill (f16 caches, and the f32
sources staged inside the kernel), and the decode scratch's growth around a
captured graph."""
import os

import numpy as np
import pytest
import torch

import oracle
from tests.util import up, up_f16

pytestmark = pytest.mark.gpu


def _replays_match(fn, n=4):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eager = [t.clone() for t in fn()]
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            outs = fn()
    torch.cuda.current_stream().wait_stream(s)
    for i in range(n):
        # unrelated eager work and a sync between replays
        junk = torch.randn(1 << 20, device="cuda").sum()
        torch.cuda.synchronize()
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(eager, outs):
            assert torch.equal(a, b), f"replay {i} differs from the eager result"
        del junk


@pytest.mark.parametrize("two_phase", ["0", "1"])
def test_decode_graph_replays(gpu, two_phase, monkeypatch):
    from ttsxabe_amd.gpu import DecodeScratch, TiledCache16
    monkeypatch.setenv("LLMTIE_DECODE_TWO_PHASE", two_phase)
    heads, kv, hd, tk, cap = 32, 8, 128, 4000, 4096
    q = up(oracle.seq(heads * hd, 1))
    k = up_f16(oracle.seq(kv * cap * hd, 2))
    v = up_f16(oracle.seq(kv * cap * hd, 3))
    t = TiledCache16(kv, hd, cap)
    gpu.t16_from_ref(k, v, t, tk)
    s1, s2 = DecodeScratch(), DecodeScratch()
    _replays_match(lambda: [gpu.attn_decode_f16(q, k, v, heads, kv, hd, tk, cap, 0.088, False, s1),
                            gpu.attn_decode_t16(q, t, heads, tk, 0.088, False, s2)])


def test_prefill_graph_replays(gpu):
    heads, kv, hd, tq, cap = 32, 8, 128, 300, 512
    q = up(oracle.seq(tq * heads * hd, 4))
    k16 = up_f16(oracle.seq(kv * cap * hd, 5))
    v16 = up_f16(oracle.seq(kv * cap * hd, 6))
    k32 = up(oracle.seq(kv * cap * hd, 5))
    v32 = up(oracle.seq(kv * cap * hd, 6))
    _replays_match(lambda: [gpu.flash_attn_f16(q, k16, v16, tq, 0, heads, kv, hd, cap, 0.088, True),
                            gpu.flash_attn(q, k32, v32, tq, 0, heads, kv, hd, cap, 0.088, True)])


def test_batched_q8_decode_graph_replays(gpu):
    """The stream-K decode: its mergers leave the arrival counters at zero
    in the kernel, so every replay starts clean (scratch grown by the eager
    call first)."""
    from ttsxabe_amd.gpu import DecodeScratch, KvCacheQ8
    from tests.test_q8_decode_gpu import load, random_q8_cache
    hd, heads, kv, slots, cap = 128, 32, 8, 6, 1024
    cache = KvCacheQ8(slots, kv, hd, cap)
    load(cache, *random_q8_cache(slots, kv, hd, cap, 31))
    tk = up(np.array([1000, 33, 517, 1024, 260], np.int32), torch.int32)
    slot = up(np.array([5, 0, 2, 2, 3], np.int32), torch.int32)
    q = up(oracle.normal(5 * heads * hd, 32))
    s = DecodeScratch()
    _replays_match(lambda: [gpu.attn_decode_q8_batch(q, cache, tk, slot, 1024, heads, hd ** -0.5, False, s)])


def test_encoder_rows_graph_replays(gpu):
    t, heads, hd = 1500, 20, 64
    qkv = up(oracle.seq(t * 3 * heads * hd, 7))
    _replays_match(lambda: [gpu.flash_attn_rows(qkv, t, heads, hd, 0.125)])


def test_scratch_growth_keeps_an_earlier_graph_valid(gpu):
    """A graph captured with a small scratch, then an eager call that grows
    the scratch: the old buffers stay allocated, so the old graph still
    replays to its eager result; growth inside a capture is refused by name."""
    from ttsxabe_amd.gpu import DecodeScratch, ScratchGrowthInCapture
    heads, kv, hd, cap = 32, 8, 128, 8192
    q = up(oracle.seq(heads * hd, 21))
    k = up_f16(oracle.seq(kv * cap * hd, 22))
    v = up_f16(oracle.seq(kv * cap * hd, 23))
    s = DecodeScratch()
    small = lambda: [gpu.attn_decode_f16(q, k, v, heads, kv, hd, 1000, cap, 0.088, False, s)]
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        eager = [t.clone() for t in small()]
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            outs = small()
        # a larger call on a fresh scratch inside a capture: refused, nothing launched
        g2 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g2, stream=st):
            with pytest.raises(ScratchGrowthInCapture):
                gpu.attn_decode_f16(q, k, v, heads, kv, hd, 8000, cap, 0.088, False, DecodeScratch())
            keep = q * 2.0  # the graph is not empty
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    # grow the scratch eagerly: a longer context, then twice the kv heads
    for tk, h, kvh in ((8000, heads, kv), (2000, 64, 16)):
        kk = up_f16(oracle.seq(kvh * cap * hd, 24))
        gpu.attn_decode_f16(up(oracle.seq(h * hd, 25)), kk, kk, h, kvh, hd, tk, cap, 0.088, False, s)
    torch.cuda.synchronize()
    for i in range(3):
        outs[0].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(eager[0], outs[0]), f"replay {i} after growth differs"
