"""Batched decode over the GGUF Q8_0 KV cache (no reference counterpart).

Pinned by the dequant closed form (crates/llmtie-gguf/src/dequant.rs:180-185)
plus the reference's f32 decode chain (crates/llmtie-cuda/tests/kernels.rs:
2733-2780) on the dequantised cache, at the decode bar of 2e-5 of full scale
(against the exact f64 value, and against the chain with its own error added).
"""
import numpy as np
import pytest
import torch

import oracle
from tests import tiled
from tests.util import down, full_scale_err, up

pytestmark = pytest.mark.gpu


def random_q8_cache(slots, kv, hd, cap, seed):
    n = slots * kv * cap * hd
    kc = (oracle.uniform_int(n, seed, -127, 127)).astype(np.int8)
    vc = (oracle.uniform_int(n, seed + 1, -127, 127)).astype(np.int8)
    ks = oracle.f32_to_f16(np.abs(oracle.normal(n // 32, seed + 2)) * np.float32(0.02))
    vs = oracle.f32_to_f16(np.abs(oracle.normal(n // 32, seed + 3)) * np.float32(0.02))
    return kc, ks, vc, vs


def load(cache, kc, ks, vc, vs):
    packed = tiled.pack_q8(kc, ks, vc, vs, cache.slots, cache.kv_heads, cache.head_dim, cache.cap)
    cache.data.copy_(torch.from_numpy(packed))


def dequant_seq(kc, ks, vc, vs, slot, kv, hd, cap):
    nb = hd // 32
    kq = kc.reshape(-1, kv, cap, hd)[slot].astype(np.float32)
    kd = oracle.f16_to_f32(ks).reshape(-1, kv, cap, nb)[slot]
    k = (kq.reshape(kv, cap, nb, 32) * kd[..., None]).reshape(kv, cap, hd)
    vq = vc.reshape(-1, kv, hd, cap)[slot].astype(np.float32)
    vd = oracle.f16_to_f32(vs).reshape(-1, kv, cap, nb)[slot]
    vscale = np.repeat(vd, 32, axis=2).transpose(0, 2, 1)  # [kv][hd][cap]
    v = vq * vscale
    return np.ascontiguousarray(k, np.float32).ravel(), np.ascontiguousarray(v, np.float32).ravel()


@pytest.mark.parametrize("hd,heads,kv,scale_q", [(128, 32, 8, False), (64, 20, 20, True), (128, 8, 8, False)])
def test_batched_q8_decode_matches_the_chain_on_the_dequantised_cache(gpu, hd, heads, kv, scale_q):
    from ttsxabe_amd.gpu import DecodeScratch, KvCacheQ8
    slots, cap, nseq = 6, 1024, 5
    kc, ks, vc, vs = random_q8_cache(slots, kv, hd, cap, 900 + hd)
    cache = KvCacheQ8(slots, kv, hd, cap)
    load(cache, kc, ks, vc, vs)
    tk = np.array([1, 33, 1000, 257, 1024], np.int32)
    slot = np.array([5, 0, 2, 2, 3], np.int32)
    q = oracle.normal(nseq * heads * hd, 77)
    scale = hd ** -0.5
    s = DecodeScratch()
    got1 = down(gpu.attn_decode_q8_batch(up(q), cache, up(tk, torch.int32), up(slot, torch.int32), 1024, heads,
                                         scale, scale_q, s))
    got2 = down(gpu.attn_decode_q8_batch(up(q), cache, up(tk, torch.int32), up(slot, torch.int32), 1024, heads,
                                         scale, scale_q, s))
    assert np.array_equal(got1, got2)
    n = heads * hd
    want = oracle.decode_q8_batch(q, kc, ks, vc, vs, tk, slot, heads, kv, hd, cap, scale, scale_q)
    for i in range(nseq):
        k, v = dequant_seq(kc, ks, vc, vs, slot[i], kv, hd, cap)
        exact = oracle.decode_f64(q[i * n:(i + 1) * n], k, v, heads, kv, hd, int(tk[i]), cap, scale, scale_q)
        chain = want[i * n:(i + 1) * n]
        own = full_scale_err(exact, chain)
        g = got1[i * n:(i + 1) * n]
        # One f16 rounding of P * d_v on the value side (about 2^-12 of full
        # scale), far inside the 8-bit quantisation of the cache itself.
        assert full_scale_err(exact, g) < 1e-3, f"seq {i}"
        assert full_scale_err(chain, g) < 1e-3 + own, f"seq {i}"


def test_a_mis_described_sequence_gets_nan_and_its_neighbours_do_not(gpu):
    from ttsxabe_amd.gpu import DecodeScratch, KvCacheQ8
    hd, heads, kv, slots, cap = 128, 8, 2, 2, 64
    cache = KvCacheQ8(slots, kv, hd, cap)
    load(cache, *random_q8_cache(slots, kv, hd, cap, 5))
    tk = up(np.array([10, 10, 0], np.int32), torch.int32)
    slot = up(np.array([0, 7, 1], np.int32), torch.int32)
    q = up(oracle.normal(3 * heads * hd, 3))
    out = down(gpu.attn_decode_q8_batch(q, cache, tk, slot, 64, heads, 0.1, False, DecodeScratch()))
    n = heads * hd
    assert np.isfinite(out[:n]).all()
    assert np.isnan(out[n:]).all()


def test_q8_refusals(gpu):
    from ttsxabe_amd.gpu import CacheOverrun, DecodeScratch, KvCacheQ8, RaggedBlock, UnsupportedAttention
    cache = KvCacheQ8(1, 2, 128, 64)
    q = torch.zeros(8 * 128, device="cuda")
    tk = torch.ones(1, dtype=torch.int32, device="cuda")
    s = DecodeScratch()
    with pytest.raises(CacheOverrun):
        gpu.attn_decode_q8_batch(q, cache, tk, tk * 0, 65, 8, 0.1, False, s)
    with pytest.raises(UnsupportedAttention):
        gpu.attn_decode_q8_batch(q, cache, tk, tk * 0, 64, 7, 0.1, False, s)
    short = KvCacheQ8(1, 2, 128, 64)
    short.data = short.data[:100]
    from ttsxabe_amd.gpu import SliceOverrun
    with pytest.raises(SliceOverrun):
        gpu.attn_decode_q8_batch(q, short, tk, tk * 0, 10, 8, 0.1, False, s)


def check_batch(gpu, hd, heads, kv, slots, cap, tk, slot, seed, scale_q=False):
    """The batched decode of (tk, slot) against the exact f64 attention on
    the dequantised cache, and bit-identical on a repeated call."""
    from ttsxabe_amd.gpu import DecodeScratch, KvCacheQ8
    kc, ks, vc, vs = random_q8_cache(slots, kv, hd, cap, seed)
    cache = KvCacheQ8(slots, kv, hd, cap)
    load(cache, kc, ks, vc, vs)
    nseq = len(tk)
    q = oracle.normal(nseq * heads * hd, seed + 7)
    scale = hd ** -0.5
    s = DecodeScratch()
    max_tk = int(max(tk))
    call = lambda: down(gpu.attn_decode_q8_batch(up(q), cache, up(tk, torch.int32), up(slot, torch.int32), max_tk,
                                                 heads, scale, scale_q, s))
    got = call()
    assert np.array_equal(got, call())
    n = heads * hd
    for i in range(nseq):
        k, v = dequant_seq(kc, ks, vc, vs, slot[i], kv, hd, cap)
        exact = oracle.decode_f64(q[i * n:(i + 1) * n], k, v, heads, kv, hd, int(tk[i]), cap, scale, scale_q)
        assert full_scale_err(exact, got[i * n:(i + 1) * n]) < 1e-3, f"seq {i} (tk {tk[i]})"


def test_many_one_block_heads(gpu):
    """64 sequences of 1..40 keys: every wave's range holds many whole heads
    and segments that begin while another segment's queries are pending."""
    tk = (oracle.uniform_int(64, 31, 1, 40)).astype(np.int32)
    check_batch(gpu, 128, 32, 8, 64, 64, tk, np.arange(64, dtype=np.int32)[::-1].copy(), 40)


def test_one_long_sequence_many_contributors(gpu):
    """One sequence of 8191 keys: every head is shared by more waves than one
    merge batch holds."""
    check_batch(gpu, 128, 32, 8, 1, 8192, np.array([8191], np.int32), np.array([0], np.int32), 41)


def test_ragged_mix_and_head_width_64(gpu):
    tk = (oracle.uniform_int(33, 32, 1, 3000)).astype(np.int32)
    check_batch(gpu, 64, 16, 4, 33, 3008, tk, np.arange(33, dtype=np.int32), 42, scale_q=True)


def test_more_than_64_sequences_take_the_planned_grid(gpu):
    tk = (oracle.uniform_int(70, 33, 1, 300)).astype(np.int32)
    check_batch(gpu, 128, 8, 2, 70, 320, tk, np.arange(70, dtype=np.int32), 43)


@pytest.mark.parametrize("hd,heads,kv", [(128, 16, 1), (64, 8, 8), (128, 64, 4)])
def test_group_widths(gpu, hd, heads, kv):
    """GQA groups of 16 (the largest query buffers) and 1 (MHA)."""
    tk = (oracle.uniform_int(9, 34 + heads, 1, 700)).astype(np.int32)
    check_batch(gpu, hd, heads, kv, 9, 704, tk, np.arange(9, dtype=np.int32)[::-1].copy(), 44 + heads)
