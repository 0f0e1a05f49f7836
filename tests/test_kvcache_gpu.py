"""KV-cache producers: RoPE, append, fused rotate+append, growth, Q8_0.

Mirrors crates/llmtie-cuda/tests/kernels.rs:1443-1539 (rope at every offset,
Llama-3 factors, no-divisor bit equality), :1919-2069 (the fused rotate+cache
is the chain), :2144-2240 (growth re-strides every head; refusals). The Q8_0
producers have no reference test; they are held to ggml's quantizer (oracle)
bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import tiled
from tests.util import down, full_scale_err, up, up_f16

pytestmark = pytest.mark.gpu

F32EPS = float(np.finfo(np.float32).eps)
LLAMA3_DIV = np.array([1.0] * 29 + [1.207484, 1.553415, 2.026313, 2.69453, 3.684253, 5.257327] + [8.0] * 29,
                      np.float32)


@pytest.mark.parametrize("first", [0, 1, 17, 4095])
def test_rope_matches_at_every_offset(gpu, first):
    t, heads, hd = 5, 3, 128
    x = oracle.seq(t * heads * hd, 75)
    want = oracle.rope(x, t, heads, hd, 10000.0, first)
    dev = up(x)
    gpu.rope(dev, 0, t, heads, hd, 10000.0, first)
    assert full_scale_err(want, down(dev)) < 1e-5 + first * F32EPS


@pytest.mark.parametrize("first", [0, 1, 4095])
def test_scaled_rope_matches_the_twin_with_llama3_factors(gpu, first):
    t, heads, hd = 4, 3, 128
    x = oracle.seq(t * heads * hd, 91)
    want = oracle.rope(x, t, heads, hd, 500000.0, first, LLAMA3_DIV)
    dev = up(x)
    gpu.rope_scaled(dev, 0, up(LLAMA3_DIV), t, heads, hd, 500000.0, first)
    assert full_scale_err(want, down(dev)) < 1e-5 + first * F32EPS


def test_scaled_rope_with_no_divisor_is_the_unscaled_one(gpu):
    t, heads, hd = 3, 2, 64
    x = oracle.seq(t * heads * hd, 12)
    a, b = up(x), up(x)
    gpu.rope(a, 0, t, heads, hd, 10000.0, 7)
    gpu.rope_scaled(b, 0, None, t, heads, hd, 10000.0, 7)
    assert np.array_equal(down(a), down(b))


@pytest.mark.parametrize("pos,scaled", [(0, True), (7, False), (31, True)])
def test_the_fused_rotate_and_cache_is_the_chain_it_replaces(gpu, pos, scaled):
    heads, kv, hd, cap = 6, 2, 16, 32
    half = hd // 2
    div = np.array([1.0 if i < 5 else 8.0 for i in range(half)], np.float32)
    theta = 500000.0
    qk = oracle.seq(heads * hd + kv * hd + 5, 17)
    vv = oracle.seq(kv * hd + 3, 23)
    q_off, k_off, v_off = 0, heads * hd + 5, 3
    kfill = oracle.seq(cap * kv * hd, 5)
    vfill = oracle.seq(cap * kv * hd, 9)
    d = up(div) if scaled else None
    # The chain: two rotations, two appends.
    cqk, cv = up(qk), up(vv)
    ck, cvc = up_f16(kfill), up_f16(vfill)
    gpu.rope_scaled(cqk, q_off, d, 1, heads, hd, theta, pos)
    gpu.rope_scaled(cqk, k_off, d, 1, kv, hd, theta, pos)
    gpu.cache_append_f16(cqk, k_off, ck, 1, kv, hd, cap, pos, False)
    gpu.cache_append_f16(cv, v_off, cvc, 1, kv, hd, cap, pos, True)
    # The fused kernel.
    fqk, fv = up(qk), up(vv)
    fk, fvc = up_f16(kfill), up_f16(vfill)
    gpu.rope_cache_f16(fqk, q_off, fqk, k_off, fv, v_off, d, heads, kv, hd, theta, pos, fk, fvc, cap)
    assert np.array_equal(down(cqk)[:heads * hd], down(fqk)[:heads * hd]), "q"
    assert np.array_equal(down(ck).view(np.uint16), down(fk).view(np.uint16)), "k cache"
    assert np.array_equal(down(cvc).view(np.uint16), down(fvc).view(np.uint16)), "v cache"
    # And the cache holds what the oracle's rotation rounds to.
    want_q = oracle.rope(qk[:heads * hd], 1, heads, hd, theta, pos, div if scaled else None)
    assert full_scale_err(want_q, down(fqk)[:heads * hd]) < 1e-5 + pos * F32EPS


@pytest.mark.parametrize("transposed", [False, True])
def test_growing_a_cache_puts_every_head_where_the_larger_capacity_wants_it(gpu, transposed):
    live, kv, hd, small, large = 5, 3, 4, 8, 16
    src = up(oracle.seq(live * kv * hd, 7))
    for f16 in (False, True):
        mk = (lambda n: torch.zeros(n, dtype=torch.float16, device="cuda")) if f16 else \
             (lambda n: torch.zeros(n, device="cuda"))
        app = gpu.cache_append_f16 if f16 else gpu.cache_append
        grow = gpu.cache_grow_f16 if f16 else gpu.cache_grow
        grew = mk(small * kv * hd)
        app(src, 0, grew, live, kv, hd, small, 0, transposed)
        moved = mk(large * kv * hd)
        grow(grew, moved, kv, hd, small, large, live, transposed)
        direct = mk(large * kv * hd)
        app(src, 0, direct, live, kv, hd, large, 0, transposed)
        assert torch.equal(moved, direct)


def test_a_growth_that_shrinks_or_overruns_is_refused(gpu):
    from ttsxabe_amd.gpu import CacheOverrun
    kv, hd, small, large = 2, 4, 8, 16
    src = torch.zeros(small * kv * hd, device="cuda")
    dst = torch.zeros(large * kv * hd, device="cuda")
    with pytest.raises(CacheOverrun):
        gpu.cache_grow(src, dst, kv, hd, small, large, small + 1, False)
    smaller = torch.zeros(small * kv * hd, device="cuda")
    with pytest.raises(CacheOverrun):
        gpu.cache_grow(src, smaller, kv, hd, large, small, 4, False)


def test_an_offset_past_the_end_of_the_source_is_refused(gpu):
    from ttsxabe_amd.gpu import SliceOverrun
    t, heads, hd = 2, 2, 8
    x = torch.zeros(t * heads * hd, device="cuda")
    with pytest.raises(SliceOverrun):
        gpu.rope(x, 1, t, heads, hd, 10000.0, 0)
    dst = torch.zeros(8 * heads * hd, device="cuda")
    with pytest.raises(SliceOverrun):
        gpu.cache_append(x, 1, dst, t, heads, hd, 8, 0, False)


def _plain_q8(slots, kv, hd, cap):
    n = slots * kv * cap * hd
    return (np.zeros(n, np.int8), np.zeros(n // 32, np.uint16), np.zeros(n, np.int8), np.zeros(n // 32, np.uint16))


@pytest.mark.parametrize("hd", [64, 128])
def test_q8_append_is_ggml_quantize(gpu, hd):
    from ttsxabe_amd.gpu import KvCacheQ8
    slots, kv, cap, n, past, slot = 3, 2, 64, 9, 5, 1
    cache = KvCacheQ8(slots, kv, hd, cap)
    k = oracle.seq(n * kv * hd, 401) * np.float32(3.0)
    v = oracle.seq(n * kv * hd, 402)
    k[:32] = 0.0  # an all-zero block: scale 0, codes 0
    v[5] = 127.0 * 0.5 / 10.0  # a value sitting near a rounding tie
    gpu.kv_q8_append(up(k), 0, up(v), 0, cache, slot, n, past)
    kc, ks, vc, vs = _plain_q8(slots, kv, hd, cap)
    kc4 = kc.reshape(slots, kv, cap, hd)
    vc4 = vc.reshape(slots, kv, hd, cap)
    ks4 = ks.reshape(slots, kv, cap, hd // 32)
    vs4 = vs.reshape(slots, kv, cap, hd // 32)
    for t in range(n):
        for h in range(kv):
            row = (t * kv + h) * hd
            c, sc = oracle.q8_0_quantize(k[row:row + hd])
            kc4[slot, h, past + t] = c
            ks4[slot, h, past + t] = sc
            c, sc = oracle.q8_0_quantize(v[row:row + hd])
            vc4[slot, h, :, past + t] = c
            vs4[slot, h, past + t] = sc
    want = tiled.pack_q8(kc, ks, vc, vs, slots, kv, hd, cap)
    assert np.array_equal(down(cache.data), want)


def test_the_q8_rotate_and_cache_is_rope_then_q8_append(gpu):
    from ttsxabe_amd.gpu import KvCacheQ8
    heads, kv, hd, cap, slots, slot, pos = 8, 2, 128, 64, 2, 1, 37
    theta = 500000.0
    q = oracle.seq(heads * hd, 31)
    k = oracle.seq(kv * hd, 32)
    v = oracle.seq(kv * hd, 33)
    div = up(LLAMA3_DIV)
    a = KvCacheQ8(slots, kv, hd, cap)
    qa, ka = up(q), up(k)
    gpu.rope_scaled(qa, 0, div, 1, heads, hd, theta, pos)
    gpu.rope_scaled(ka, 0, div, 1, kv, hd, theta, pos)
    gpu.kv_q8_append(ka, 0, up(v), 0, a, slot, 1, pos)
    b = KvCacheQ8(slots, kv, hd, cap)
    qb = up(q)
    gpu.rope_cache_q8(qb, 0, up(k), 0, up(v), 0, div, heads, theta, pos, b, slot)
    assert torch.equal(qa, qb)
    assert torch.equal(a.data, b.data)


@pytest.mark.parametrize("hd", [64, 128])
def test_tiled_f16_producers_are_the_reference_producers_repacked(gpu, hd):
    """t16_append / t16_rope_cache / t16_from_ref write exactly the reference
    layout's bits, repacked as the numpy packer says; t16_grow re-strides."""
    from ttsxabe_amd.gpu import TiledCache16
    heads, kv, cap, n, past = 8, 2, 100, 37, 3
    theta = 500000.0
    src_k = up(oracle.seq(n * kv * hd, 51))
    src_v = up(oracle.seq(n * kv * hd, 52))
    rk = torch.zeros(kv * cap * hd, dtype=torch.float16, device="cuda")
    rv = torch.zeros(kv * cap * hd, dtype=torch.float16, device="cuda")
    gpu.cache_append_f16(src_k, 0, rk, n, kv, hd, cap, past, False)
    gpu.cache_append_f16(src_v, 0, rv, n, kv, hd, cap, past, True)
    t = TiledCache16(kv, hd, cap)
    gpu.t16_append(src_k, 0, t, n, past, False)
    gpu.t16_append(src_v, 0, t, n, past, True)
    want = tiled.pack_t16(down(rk).view(np.uint16), down(rv).view(np.uint16), kv, hd, cap)
    assert np.array_equal(down(t.data).view(np.uint16), want)
    # The device repacker agrees with the numpy packer.
    t2 = TiledCache16(kv, hd, cap)
    gpu.t16_from_ref(rk, rv, t2, past + n)
    assert torch.equal(t.data, t2.data)
    # Fused rotate + cache at one position.
    q = oracle.seq(heads * hd, 53)
    kx = oracle.seq(kv * hd, 54)
    vx = oracle.seq(kv * hd, 55)
    qa, qb = up(q), up(q)
    gpu.rope_cache_f16(qa, 0, up(kx), 0, up(vx), 0, None, heads, kv, hd, theta, past + n, rk, rv, cap)
    gpu.t16_rope_cache(qb, 0, up(kx), 0, up(vx), 0, None, heads, theta, past + n, t)
    assert torch.equal(qa, qb)
    want = tiled.pack_t16(down(rk).view(np.uint16), down(rv).view(np.uint16), kv, hd, cap)
    assert np.array_equal(down(t.data).view(np.uint16), want)
    # Growth: every head's blocks land where the larger capacity wants them.
    big = TiledCache16(kv, hd, 2 * cap)
    gpu.t16_grow(t, big, past + n + 1)
    rk2 = torch.zeros(kv * 2 * cap * hd, dtype=torch.float16, device="cuda")
    rv2 = torch.zeros(kv * 2 * cap * hd, dtype=torch.float16, device="cuda")
    gpu.cache_grow_f16(rk, rk2, kv, hd, cap, 2 * cap, past + n + 1, False)
    gpu.cache_grow_f16(rv, rv2, kv, hd, cap, 2 * cap, past + n + 1, True)
    want = tiled.pack_t16(down(rk2).view(np.uint16), down(rv2).view(np.uint16), kv, hd, 2 * cap, live=past + n + 1)
    got = down(big.data).view(np.uint16)
    # Positions past `live` inside the last copied block are carried along
    # whole (they were zero in the source), so the images agree everywhere.
    assert np.array_equal(got, want)


def _ref_scatter(fill, vals, kv, hd, cap, past, transposed):
    """Rows [n][kv][hd] written at positions past.. of K [kv][cap][hd]
    (transposed: V^T [kv][hd][cap]) over `fill`, in numpy."""
    out = fill.copy()
    n = vals.shape[0]
    if transposed:
        out.reshape(kv, hd, cap)[:, :, past:past + n] = vals.transpose(1, 2, 0)
    else:
        out.reshape(kv, cap, hd)[:, past:past + n, :] = vals.transpose(1, 0, 2)
    return out


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("transposed", [False, True])
def test_append_writes_the_reference_layout_bit_for_bit(gpu, f16, transposed):
    """cache_append / cache_append_f16 against a numpy scatter of the rows
    (rounded by the oracle's RNE f16 for the f16 cache) into the reference
    layouts, every other position untouched (kernels.rs:1919-2069, 3013,
    2849)."""
    n, kv, hd, cap, past, off = 7, 3, 64, 40, 9, 5
    src = oracle.seq(off + n * kv * hd, 301)
    fill = oracle.seq(kv * cap * hd, 302)
    rows = src[off:].reshape(n, kv, hd)
    if f16:
        want = _ref_scatter(oracle.f32_to_f16(fill), oracle.f32_to_f16(rows.ravel()).reshape(n, kv, hd), kv, hd, cap,
                            past, transposed)
        dst = up_f16(fill)
        gpu.cache_append_f16(up(src), off, dst, n, kv, hd, cap, past, transposed)
        assert np.array_equal(down(dst).view(np.uint16), want)
    else:
        want = _ref_scatter(fill, rows, kv, hd, cap, past, transposed)
        dst = up(fill)
        gpu.cache_append(up(src), off, dst, n, kv, hd, cap, past, transposed)
        assert np.array_equal(down(dst).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("transposed", [False, True])
def test_growth_restrides_the_reference_layout_bit_for_bit(gpu, f16, transposed):
    """cache_grow / cache_grow_f16 against numpy: the first `live` positions of
    every head (every value row, transposed) move to the larger stride, the
    rest of the destination is untouched (kernels.rs:2144-2240, 3086, 3152)."""
    kv, hd, cap, new_cap, live = 3, 64, 24, 56, 19
    src = oracle.seq(kv * cap * hd, 311)
    fill = oracle.seq(kv * new_cap * hd, 312)
    if f16:
        src_b, fill_b = oracle.f32_to_f16(src), oracle.f32_to_f16(fill)
    else:
        src_b, fill_b = src.view(np.uint32), fill.view(np.uint32)
    want = fill_b.copy()
    if transposed:
        want.reshape(kv * hd, new_cap)[:, :live] = src_b.reshape(kv * hd, cap)[:, :live]
    else:
        want.reshape(kv, new_cap * hd)[:, :live * hd] = src_b.reshape(kv, cap * hd)[:, :live * hd]
    if f16:
        d_src, d_dst = up_f16(src), up_f16(fill)
        gpu.cache_grow_f16(d_src, d_dst, kv, hd, cap, new_cap, live, transposed)
        assert np.array_equal(down(d_dst).view(np.uint16), want)
    else:
        d_src, d_dst = up(src), up(fill)
        gpu.cache_grow(d_src, d_dst, kv, hd, cap, new_cap, live, transposed)
        assert np.array_equal(down(d_dst).view(np.uint32), want)


def test_rope_cache_writes_the_reference_layout(gpu):
    """rope_cache_f16 against the oracle: the V row lands at `pos` of V^T as
    RNE f16 bit for bit; the K row is the oracle's rotation rounded to f16,
    within one f16 step (the rotation itself matches to ~1e-6 relative, which
    can move a value across a rounding boundary); q is rotated in place; all
    other positions are untouched (kernels.rs:1919-2069, 5334)."""
    heads, kv, hd, cap, pos = 8, 2, 128, 48, 29
    theta = 500000.0
    q = oracle.seq(heads * hd, 321)
    k = oracle.seq(kv * hd, 322)
    v = oracle.seq(kv * hd, 323)
    kfill = oracle.seq(kv * cap * hd, 324)
    vfill = oracle.seq(kv * cap * hd, 325)
    dq, dk, dvc = up(q), up_f16(kfill), up_f16(vfill)
    gpu.rope_cache_f16(dq, 0, up(k), 0, up(v), 0, None, heads, kv, hd, theta, pos, dk, dvc, cap)
    want_v = _ref_scatter(oracle.f32_to_f16(vfill), oracle.f32_to_f16(v).reshape(1, kv, hd), kv, hd, cap, pos, True)
    assert np.array_equal(down(dvc).view(np.uint16), want_v)
    kr = oracle.rope(k, 1, kv, hd, theta, pos)
    want_k = _ref_scatter(oracle.f32_to_f16(kfill), oracle.f32_to_f16(kr).reshape(1, kv, hd), kv, hd, cap, pos, False)
    got_k = down(dk).view(np.uint16)
    other = np.ones((kv, cap, hd), bool)
    other[:, pos, :] = False
    other = other.ravel()
    assert np.array_equal(got_k[other], want_k[other])
    step = np.abs(got_k[~other].astype(np.int32) - want_k[~other].astype(np.int32))
    assert step.max() <= 1, f"K row off by {step.max()} f16 steps"
    assert full_scale_err(oracle.rope(q, 1, heads, hd, theta, pos), down(dq)) < 1e-5 + pos * F32EPS
