"""Pins the CPU oracle (oracle/oracle.c) before any GPU test trusts it.

Each oracle function is checked against something that does not share its
code: numpy's IEEE float16, the committed known-answer vectors of
tests/golden/known_answers.json (made by tests/golden/make_golden.py from the
reference's definitions with Python big integers and exact arithmetic), f64
closed forms written vectorised in numpy (a different formulation from the
oracle's scalar loops), and invariants chosen so that a plausible slip -- a
swapped cache index, tk read as cap, a dropped scale, a wrong rotation sign,
a transposed V, round-half-even where the reference rounds away from zero --
fails at least one of them. CPU only.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import scipy.special
import scipy.stats

import oracle

GOLD = json.loads((Path(__file__).resolve().parent / "golden" / "known_answers.json").read_text())
RNG = np.random.default_rng(20261201)


# --------------------------------------------------------------- binary16

def test_f16_to_f32_matches_ieee_on_every_half():
    h = np.arange(1 << 16, dtype=np.uint16)
    got = oracle.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne():
    # random bit patterns over the whole f32 range, plus every half, every
    # midpoint between adjacent halves (the ties), and the overflow edge
    bits = RNG.integers(0, 1 << 32, 400_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    halves = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((halves[:-1] + halves[1:]) / 2).astype(np.float32)
    near = np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0))
    edge = np.array([65504.0, 65519.99, 65520.0, 65536.0, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001,
                     2.0 ** -14, -0.0, np.inf, -np.inf], np.float32)
    for xs in (x, mids, near[0], near[1], edge, -mids):
        got = oracle.f32_to_f16(xs)
        with np.errstate(over="ignore"):
            want = xs.astype(np.float16)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got.view(np.float16)), nan)
        assert np.array_equal(got[~nan], want[~nan].view(np.uint16))


# ------------------------------------------------------------- generators

def test_seq_matches_big_integer_recurrence():
    for salt, want in GOLD["seq"].items():
        got = oracle.seq(len(want), int(salt))
        assert np.array_equal(got, np.asarray(want, np.float32)), salt


def test_seq_range_and_spread():
    # (s >> 40) / 2^23 * 4 - 2 with a 24-bit (s >> 40) is uniform on [-2, 6),
    # whatever the reference's doc comment ("roughly [-2, 2]") says
    x = oracle.seq(100_000, 5)
    assert x.min() >= -2.0 and x.max() < 6.0 and x.min() < -1.99 and x.max() > 5.99
    assert abs(x.mean() - 2.0) < 0.03 and abs(x.var() - 64.0 / 12.0) < 0.05


def test_normal_is_standard_normal_and_counter_based():
    x = oracle.normal(200_000, 7)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert scipy.stats.kstest(x, "norm").pvalue > 1e-4
    # element i depends only on (seed, first + i)
    assert np.array_equal(oracle.normal(100, 7, first=50), x[50:150])
    assert not np.array_equal(oracle.normal(100, 8), x[:100])


def test_uniform_int_bounds():
    x = oracle.uniform_int(50_000, 3, 256, 300)
    assert x.min() == 256 and x.max() == 300 and len(np.unique(x)) == 45


# --------------------------------------------------------------------- RoPE

def rope_closed_form(x, t, heads, hd, theta, first, div=None):
    """(a + ib) * exp(i * pos * inv) per pair (i, i + hd/2), in f64."""
    x = np.asarray(x, np.float64).reshape(t, heads, hd)
    half = hd // 2
    inv = theta ** (-2.0 * np.arange(half) / hd)
    if div is not None:
        inv = inv / np.asarray(div, np.float64)
    ang = (first + np.arange(t))[:, None] * inv[None, :]
    z = (x[..., :half] + 1j * x[..., half:]) * np.exp(1j * ang)[:, None, :]
    return np.concatenate([z.real, z.imag], axis=-1).ravel()


@pytest.mark.parametrize("hd,theta,first", [(64, 10_000.0, 0), (128, 500_000.0, 3), (64, 10_000.0, 40)])
def test_rope_closed_form(hd, theta, first):
    t, heads = 5, 3
    x = oracle.seq(t * heads * hd, 11)
    got = oracle.rope(x, t, heads, hd, theta, first)
    want = rope_closed_form(x, t, heads, hd, theta, first)
    # f32 angle and f32 sin/cos: error grows with the angle, ~|pos| * 2^-24
    assert np.abs(got - want).max() < 2e-5 * (first + t)


def test_rope_identity_at_zero_and_norm_preserved():
    t, heads, hd = 1, 4, 128
    x = oracle.seq(t * heads * hd, 12)
    assert np.array_equal(oracle.rope(x, t, heads, hd, 500_000.0, 0), x)
    t = 64
    x = oracle.seq(t * heads * hd, 13)
    y = oracle.rope(x, t, heads, hd, 500_000.0, 4000).reshape(t, heads, hd).astype(np.float64)
    x = x.reshape(t, heads, hd).astype(np.float64)
    nx = x[..., :64] ** 2 + x[..., 64:] ** 2
    ny = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert np.abs(nx - ny).max() < 1e-5 * max(1.0, nx.max())


def test_rope_divisor():
    t, heads, hd = 3, 2, 64
    x = oracle.seq(t * heads * hd, 14)
    assert np.array_equal(oracle.rope(x, t, heads, hd, 10_000.0, 9, np.ones(32, np.float32)),
                          oracle.rope(x, t, heads, hd, 10_000.0, 9))
    div = np.linspace(1.0, 8.0, 32).astype(np.float32)
    got = oracle.rope(x, t, heads, hd, 10_000.0, 9, div)
    assert np.abs(got - rope_closed_form(x, t, heads, hd, 10_000.0, 9, div)).max() < 1e-4


# ------------------------------------------------------------------ decode

def decode_np(q, k, v, heads, kv, hd, tk, cap, scale):
    """Vectorised f64 decode: q [heads, hd], k [kv, cap, hd], v [kv, hd, cap]."""
    g = heads // kv
    q = np.asarray(q, np.float64).reshape(kv, g, hd)
    k = np.asarray(k, np.float64).reshape(kv, cap, hd)[:, :tk]
    v = np.asarray(v, np.float64).reshape(kv, hd, cap)[:, :, :tk]
    s = np.einsum("hgd,htd->hgt", q, k) * float(np.float32(scale))  # the f32 scale the oracle is given
    p = scipy.special.softmax(s, axis=-1)
    return np.einsum("hgt,hdt->hgd", p, v).ravel()


def test_decode_hand_case():
    c = GOLD["decode_hand"]
    args = (c["heads"], c["kv"], c["hd"], c["tk"], c["cap"], c["scale"])
    want = np.asarray(c["out"])
    assert np.abs(oracle.decode_ref(c["q"], c["k"], c["v"], *args, False) - want).max() < 1e-6
    assert np.abs(oracle.decode_ref(c["q"], c["k"], c["v"], *args, True) - want).max() < 1e-6
    assert np.abs(oracle.decode_f64(c["q"], c["k"], c["v"], *args) - want).max() < 1e-14


@pytest.mark.parametrize("heads,kv,hd,tk,cap,scale_q", [
    (8, 2, 128, 200, 256, False), (6, 6, 64, 37, 448, True), (32, 8, 128, 1000, 1024, False)])
def test_decode_closed_form(heads, kv, hd, tk, cap, scale_q):
    q = oracle.seq(heads * hd, 1) - 2.0
    k = oracle.seq(kv * cap * hd, 2)
    v = oracle.seq(kv * hd * cap, 3)
    # capacity past tk holds NaN: reading it would poison the result
    k.reshape(kv, cap, hd)[:, tk:] = np.nan
    v.reshape(kv, hd, cap)[:, :, tk:] = np.nan
    want = decode_np(q, k, v, heads, kv, hd, tk, cap, 0.11)
    got = oracle.decode_ref(q, k, v, heads, kv, hd, tk, cap, 0.11, scale_q)
    # the f32 chain (sequential sums) stays well inside the reference's own
    # 2e-5-of-full-scale decode bar
    assert np.abs(got - want).max() < 5e-6 * np.abs(want).max()
    assert np.abs(oracle.decode_f64(q, k, v, heads, kv, hd, tk, cap, 0.11) - want).max() < 1e-12


def test_decode_invariants():
    heads, kv, hd, cap = 4, 2, 64, 96
    k = oracle.seq(kv * cap * hd, 4)
    v = oracle.seq(kv * hd * cap, 5)
    vv = v.reshape(kv, hd, cap).astype(np.float64)
    # zero query: uniform weights over the tk live keys -> the mean of V
    got = oracle.decode_ref(np.zeros(heads * hd, np.float32), k, v, heads, kv, hd, 50, cap, 0.3, False)
    want = np.repeat(vv[:, :, :50].mean(-1), heads // kv, axis=0).ravel()
    assert np.abs(got - want).max() < 1e-6
    # one key: the output is that key's value column exactly
    q = oracle.seq(heads * hd, 6)
    got = oracle.decode_ref(q, k, v, heads, kv, hd, 1, cap, 0.3, False)
    assert np.array_equal(got, np.repeat(vv[:, :, 0], heads // kv, axis=0).ravel().astype(np.float32))
    # every head of a group reads the same kv head
    q2 = np.tile(q.reshape(kv, 2, hd)[:, :1], (1, 2, 1)).ravel()
    got = oracle.decode_ref(q2, k, v, heads, kv, hd, 70, cap, 0.3, False).reshape(kv, 2, hd)
    assert np.array_equal(got[:, 0], got[:, 1])


def test_decode_f16_is_decode_ref_on_rounded_cache():
    heads, kv, hd, tk, cap = 8, 2, 128, 300, 320
    q = oracle.seq(heads * hd, 7)
    kb = oracle.f32_to_f16(oracle.seq(kv * cap * hd, 8))
    vb = oracle.f32_to_f16(oracle.seq(kv * hd * cap, 9))
    want = oracle.decode_ref(q, oracle.f16_to_f32(kb), oracle.f16_to_f32(vb), heads, kv, hd, tk, cap, 0.1, False)
    for threads in (1, 4):
        got = oracle.decode_f16(q, kb, vb, heads, kv, hd, tk, cap, 0.1, False, threads)
        assert np.array_equal(got, want)


# ------------------------------------------------------------------ prefill

def prefill_np(q, qs, k, v, tq, past, heads, kv, hd, cap, scale, causal, round_p):
    """Vectorised f64 prefill on f16-rounded operands; P rounded to f16 when
    round_p (the reference's value product), normaliser unrounded."""
    r16 = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float64)
    tk = past + tq
    g = heads // kv
    qq = r16(np.asarray(q, np.float32).reshape(tq, qs)[:, :heads * hd]).reshape(tq, kv, g, hd)
    kk = r16(np.asarray(k).reshape(kv, cap, hd)[:, :tk])
    vv = r16(np.asarray(v).reshape(kv, hd, cap)[:, :, :tk])
    s = np.einsum("rhgd,htd->rhgt", qq, kk) * float(np.float32(scale))
    if causal:
        mask = np.arange(tk)[None, :] > (past + np.arange(tq))[:, None]
        s = np.where(mask[:, None, None, :], -np.inf, s)
    e = np.exp(s - s.max(-1, keepdims=True))
    l = e.sum(-1, keepdims=True)
    p = r16(e) if round_p else e
    o = np.einsum("rhgt,hdt->rhgd", p, vv) / l
    return o.reshape(tq, heads * hd)


@pytest.mark.parametrize("tq,past,heads,kv,hd,cap,causal", [
    (17, 0, 4, 2, 64, 32, True), (9, 23, 4, 1, 128, 40, True), (12, 0, 3, 3, 64, 16, False)])
def test_prefill_closed_form(tq, past, heads, kv, hd, cap, causal):
    qs = heads * hd + 8  # a row stride wider than the heads
    q = oracle.seq(tq * qs, 71) * 100.0  # peaked, as the reference test makes it
    k = oracle.seq(kv * cap * hd, 72)
    v = oracle.seq(kv * hd * cap, 73)
    want, spread = oracle.prefill_ref(q, qs, k, v, tq, past, heads, kv, hd, cap, 0.125, causal, threads=2)
    want = want.reshape(tq, heads * hd)
    assert np.abs(want - prefill_np(q, qs, k, v, tq, past, heads, kv, hd, cap, 0.125, causal, True)).max() < 1e-12
    # unrounded P differs from the rounded one by at most 2^-11 relative
    exact = prefill_np(q, qs, k, v, tq, past, heads, kv, hd, cap, 0.125, causal, False)
    assert np.abs(want - exact).max() < 2.0 ** -10 * 2.0
    # spread is the probability-weighted mean distance to the average
    assert (spread >= 0).all() and spread.max() < 4.0


def test_prefill_causal_rows_ignore_later_keys():
    tq, heads, kv, hd, cap = 10, 2, 1, 64, 10
    q = oracle.seq(tq * heads * hd, 1)
    k = oracle.seq(kv * cap * hd, 2)
    v = oracle.seq(kv * hd * cap, 3)
    a, _ = oracle.prefill_ref(q, heads * hd, k, v, tq, 0, heads, kv, hd, cap, 0.2, True, threads=1)
    k2, v2 = k.copy(), v.copy()
    k2.reshape(kv, cap, hd)[:, 6:] += 1.0
    v2.reshape(kv, hd, cap)[:, :, 6:] -= 1.0
    b, _ = oracle.prefill_ref(q, heads * hd, k2, v2, tq, 0, heads, kv, hd, cap, 0.2, True, threads=1)
    a, b = a.reshape(tq, -1), b.reshape(tq, -1)
    assert np.array_equal(a[:6], b[:6]) and not np.array_equal(a[6:], b[6:])


def test_prefill_one_key_and_permutation():
    heads, kv, hd = 2, 2, 64
    q = oracle.seq(heads * hd, 4)
    k = oracle.seq(kv * 8 * hd, 5)
    v = oracle.seq(kv * hd * 8, 6)
    w, sp = oracle.prefill_ref(q, heads * hd, k, v, 1, 0, heads, kv, hd, 8, 0.2, True, threads=1)
    assert np.array_equal(w.reshape(heads, hd), oracle.through_f16(v.reshape(kv, hd, 8)[:, :, 0]))
    assert not sp.any()
    # non-causal attention is invariant under a permutation of the keys
    tq, cap = 6, 6
    q = oracle.seq(tq * heads * hd, 7)
    k = oracle.seq(kv * cap * hd, 8).reshape(kv, cap, hd)
    v = oracle.seq(kv * hd * cap, 9).reshape(kv, hd, cap)
    perm = np.array([3, 0, 5, 1, 4, 2])
    a, _ = oracle.prefill_ref(q, heads * hd, k, v, tq, 0, heads, kv, hd, cap, 0.2, False, threads=1)
    b, _ = oracle.prefill_ref(q, heads * hd, k[:, perm], v[:, :, perm], tq, 0, heads, kv, hd, cap, 0.2, False,
                              threads=1)
    assert np.abs(a - b).max() < 1e-12


def test_prefill_f32_closed_form():
    t, heads, kv, hd = 20, 4, 2, 64
    q = oracle.seq(t * heads * hd, 1) - 2.0  # centred, so f32 score rounding stays small
    k = oracle.seq(t * kv * hd, 2) - 2.0
    v = oracle.seq(t * kv * hd, 3)
    got = oracle.prefill_f32(q, k, v, t, heads, kv, hd, 0.125, True, threads=2).reshape(t, heads * hd)
    # the same through the decode closed form, one row at a time
    kk = k.reshape(t, kv, hd).transpose(1, 0, 2)
    vv = v.reshape(t, kv, hd).transpose(1, 2, 0)
    for r in range(t):
        want = decode_np(q.reshape(t, -1)[r], kk[:, :r + 1], vv[:, :, :r + 1], heads, kv, hd, r + 1, r + 1, 0.125)
        assert np.abs(got[r] - want).max() < 5e-6 * np.abs(want).max()


# --------------------------------------------------------------------- Q8_0

def test_q8_dequant_closed_form():
    codes = RNG.integers(-128, 128, 32 * 40).astype(np.int8)
    scales = oracle.f32_to_f16(np.abs(RNG.normal(0, 0.02, 40)).astype(np.float32))
    got = oracle.q8_0_dequant(codes, scales)
    want = codes.astype(np.float32) * np.repeat(scales.view(np.float16).astype(np.float32), 32)
    assert np.array_equal(got, want)


def test_q8_quantize_hand_case_rounds_half_away_from_zero():
    c = GOLD["q8_hand"]
    codes, scales = oracle.q8_0_quantize(np.asarray(c["x"], np.float32))
    assert codes.tolist() == c["codes"] and scales.tolist() == [c["scale_bits"]]


def test_q8_round_trip_error():
    x = oracle.normal(32 * 500, 3) * 0.7
    codes, scales = oracle.q8_0_quantize(x)
    d32 = np.abs(x.reshape(-1, 32)).max(1) / 127.0
    y = oracle.q8_0_dequant(codes, scales).reshape(-1, 32)
    d16 = scales.view(np.float16).astype(np.float64)
    # code error <= 1/2 step of the unrounded scale, plus the scale's own f16 rounding
    bound = d32 / 2 + np.abs(d16 - d32) * 127 + 1e-7
    assert (np.abs(y - x.reshape(-1, 32)).max(1) <= bound).all()
    assert np.abs(codes).max() <= 127 and np.abs(codes).max(axis=None) == 127


def test_twin_hand_case_rounds_half_even():
    c = GOLD["twin_hand"]
    codes, scales = oracle.twin_quantize(np.asarray(c["y"], np.float32))
    assert codes.tolist() == c["codes"] and scales.tolist() == c["scales"]


def test_decode_q8_batch_is_decode_ref_on_dequantised_cache():
    nseq, slots, heads, kv, hd, cap = 3, 4, 4, 2, 64, 96
    tk = np.array([96, 1, 50], np.int32)
    slot = np.array([2, 0, 3], np.int32)
    nb = hd // 32
    kc = RNG.integers(-127, 128, (slots, kv, cap, hd)).astype(np.int8)
    vc = RNG.integers(-127, 128, (slots, kv, hd, cap)).astype(np.int8)
    ks = oracle.f32_to_f16(np.abs(RNG.normal(0, 0.02, (slots, kv, cap, nb))).astype(np.float32))
    vs = oracle.f32_to_f16(np.abs(RNG.normal(0, 0.02, (slots, kv, cap, nb))).astype(np.float32))
    q = oracle.seq(nseq * heads * hd, 1)
    got = oracle.decode_q8_batch(q, kc, ks, vc, vs, tk, slot, heads, kv, hd, cap, 0.125, False, threads=2)
    for s in range(nseq):
        sl = slot[s]
        k = kc[sl].astype(np.float32) * np.repeat(ks[sl].view(np.float16).astype(np.float32), 32, axis=-1)
        # V codes are [hd][cap]; the scale of (dim d, position p) is vs[p][d // 32]
        vsc = np.repeat(vs[sl].view(np.float16).astype(np.float32), 32, axis=-1).transpose(0, 2, 1)
        v = vc[sl].astype(np.float32) * vsc
        want = oracle.decode_ref(q.reshape(nseq, -1)[s], k, v, heads, kv, hd, int(tk[s]), cap, 0.125, False)
        assert np.array_equal(got.reshape(nseq, -1)[s], want)


# ------------------------------------------------------------ layer stack

def test_stack_pieces_hand_cases():
    from oracle.stack import attend, rms_norm, silu_mul
    y = rms_norm(np.array([[3.0, 4.0]], np.float32), np.array([1.0, 2.0], np.float32), 0.0)
    assert np.allclose(y, [[3 / np.sqrt(12.5), 8 / np.sqrt(12.5)]], rtol=1e-6)
    assert np.array_equal(silu_mul(np.zeros(3, np.float32), np.ones(3, np.float32)), np.zeros(3, np.float32))
    assert np.allclose(silu_mul(np.array([30.0], np.float32), np.array([2.0], np.float32)), [60.0], rtol=1e-6)
    assert np.allclose(silu_mul(np.array([-1.0], np.float32), np.array([1.0], np.float32)), [-1 / (1 + np.e)])
    # zero queries: each causal row is the mean of the values it may see
    kv, hd, past, n = 1, 4, 3, 2
    k = oracle.seq(kv * 5 * hd, 1).reshape(kv, 5, hd)
    v = oracle.seq(kv * 5 * hd, 2).reshape(kv, 5, hd)
    out = attend(np.zeros((n, 2 * hd), np.float32), k, v, past, n, 2, kv, hd, 0.5)
    assert np.allclose(out[0, :hd], v[0, :4].mean(0), atol=1e-6)
    assert np.allclose(out[1, hd:], v[0, :5].mean(0), atol=1e-6)


def test_stack_with_silent_blocks_is_norm_then_head():
    from oracle.stack import CpuStack, StackConfig, random_weights
    cfg = StackConfig(vocab=64, hidden=128, heads=2, kv_heads=1, head_dim=64, ffn=64, layers=1)
    w = random_weights(cfg, 3)
    w["0.wo"][:] = 0.0   # attention contributes nothing
    w["0.wd"][:] = 0.0   # nor does the feed-forward
    s = CpuStack(cfg, w)
    got = s.forward([5, 9, 17])
    x = w["embed"][17].astype(np.float64)
    want = (x / np.sqrt((x * x).mean() + cfg.eps) * w["norm"]) @ w["lm_head"].T.astype(np.float64)
    assert np.abs(got - want).max() < 1e-4 * np.abs(want).max()
    assert s.past == 3 and s.k[0].shape == (1, 3, 64)


def test_cross_cache_ref_brute_force():
    from oracle.whisper import cross_cache_ref
    t, d, heads, layers = 3, 4, 2, 2
    rng = np.random.default_rng(5)
    enc = rng.standard_normal((t, d)).astype(np.float32)
    wk = rng.standard_normal((layers, d, d)).astype(np.float32)
    wv = rng.standard_normal((layers, d, d)).astype(np.float32)
    bv = rng.standard_normal((layers, d)).astype(np.float32)
    got = cross_cache_ref(enc, wk, wv, bv, heads)
    h16 = lambda a: np.float64(np.float16(a))
    for l in range(layers):
        for p in range(t):
            for o in range(d):
                ks = sum(h16(enc[p, i]) * h16(wk[l, o, i]) for i in range(d))
                vs = np.float32(sum(h16(enc[p, i]) * h16(wv[l, o, i]) for i in range(d))) + bv[l, o]
                h, j = divmod(o, d // heads)
                assert got[l][0][h, p, j] == np.float16(np.float32(ks)).view(np.uint16)
                assert got[l][1][h, j, p] == np.float16(np.float32(vs)).view(np.uint16)
