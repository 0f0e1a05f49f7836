"""Decode attention against the reference's decode chain on the CPU.

Mirrors crates/llmtie-cuda/tests/kernels.rs:2782-2937
(`the_fused_decode_attention_matches_the_chain`), :2071-2142 (the int8 twin)
and :3339-3463 (the row variant): the same shapes, the same `seq` inputs and
salts, the same 2e-5-of-full-scale bar, and the same bit-reproducibility
through one scratch.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.util import down, full_scale_err, up, up_f16

pytestmark = pytest.mark.gpu

# (heads, kv_heads, hd, tk, cap, f16 cache, scale on the query) - kernels.rs:2790-2822
CASES = [
    (8, 2, 128, 1, 256, True, False),
    (8, 2, 128, 63, 256, True, False),
    (8, 2, 128, 64, 256, True, False),
    (8, 2, 128, 65, 256, True, False),
    (8, 2, 128, 200, 256, True, False),
    (8, 2, 128, 256, 256, True, False),
    (4, 4, 128, 130, 512, True, False),
    (6, 6, 64, 1500, 1500, True, True),
    (6, 6, 64, 1499, 1500, True, True),
    (6, 6, 64, 37, 448, False, True),
    (6, 6, 64, 129, 448, False, True),
    (6, 6, 64, 448, 448, False, True),
    (4, 2, 128, 16500, 16512, True, False),
    (32, 8, 128, 4096, 4096, True, False),
    (32, 8, 128, 8192, 8192, True, False),
    (32, 8, 128, 7777, 8192, True, False),
    (40, 40, 128, 1500, 1536, True, False),
    (20, 20, 64, 1500, 1500, True, True),
    (8, 8, 64, 5000, 5056, False, True),
    # GQA groups of 3 (not in kernels.rs): the split merge's phase count is 5
    # at head_dim 64, not a power of two.
    (12, 4, 64, 3000, 3008, True, False),
    (6, 2, 128, 5000, 5056, True, False),
    # f32 caches at head_dim 128 (not in kernels.rs): group 1 on the VALU,
    # group 4 on the MFMA path with one block in flight per wave.
    (4, 4, 128, 300, 320, False, True),
    (8, 2, 128, 1000, 1024, False, False),
    # f32 caches at head_dim 64, group 1 (line-order fold) with capacity 2 mod
    # 4: V rows only 8-byte aligned; full blocks and a 14-key partial one.
    (5, 5, 64, 302, 450, False, False),
    (3, 3, 64, 450, 450, False, True),
    # The last block running past the capacity (capacity not a multiple of
    # 32), so its reads are clamped inside the cache: f16 with 16-byte rows,
    # f32 group 1 at head_dim 64 (16-byte rows) and 128, f32 group 4 with
    # 8-byte rows.
    (8, 2, 128, 1000, 1000, True, False),
    (4, 4, 64, 451, 452, False, True),
    (2, 2, 128, 330, 332, False, False),
    (8, 2, 128, 1001, 1002, False, False),
    # One live key, and a partial block of one key after a full one, on the
    # group-1 folds (f32 line order, f16, f32 at head_dim 128).
    (4, 4, 64, 1, 452, False, True),
    (4, 4, 64, 33, 452, False, True),
    (4, 4, 64, 33, 452, True, True),
    (2, 2, 128, 1, 64, False, False),
]


@pytest.mark.parametrize("i", range(len(CASES)))
def test_the_fused_decode_attention_matches_the_chain(gpu, i):
    from ttsxabe_amd.gpu import DecodeScratch
    heads, kv, hd, tk, cap, half, scale_q = CASES[i]
    salt = 300 + 3 * i
    q = oracle.seq(heads * hd, salt)
    k0 = oracle.seq(kv * cap * hd, salt + 1)
    v0 = oracle.seq(kv * hd * cap, salt + 2)
    k, v = (oracle.through_f16(k0), oracle.through_f16(v0)) if half else (k0, v0)
    scale = 0.11
    want = oracle.decode_ref(q, k, v, heads, kv, hd, tk, cap, scale, scale_q)
    scratch = DecodeScratch()
    dq = up(q)
    if half:
        dk, dv = up_f16(k0), up_f16(v0)
        f = gpu.attn_decode_f16
    else:
        dk, dv = up(k0), up(v0)
        f = gpu.attn_decode
    a = down(f(dq, dk, dv, heads, kv, hd, tk, cap, scale, scale_q, scratch))
    b = down(f(dq, dk, dv, heads, kv, hd, tk, cap, scale, scale_q, scratch))
    assert np.array_equal(a, b), "not reproducible through one scratch"
    if half:
        # The tiled cache holds the same halves in fragment order: the same
        # MFMA inputs in the same slots, so the same bits out.
        from ttsxabe_amd.gpu import TiledCache16
        t = TiledCache16(kv, hd, cap)
        gpu.t16_from_ref(dk, dv, t, tk)
        c_ = down(gpu.attn_decode_t16(dq, t, heads, tk, scale, scale_q, scratch))
        assert np.array_equal(a, c_), "tiled cache differs from the reference layout"
    exact = oracle.decode_f64(q, k, v, heads, kv, hd, tk, cap, scale, scale_q)
    own = full_scale_err(exact, want)  # the f32 chain's own rounding
    err_exact = full_scale_err(exact, a)
    err = full_scale_err(want, a)
    assert err_exact < 2e-5, f"case {CASES[i]}: {err_exact:.3e} of full scale from the exact value"
    assert err < 2e-5 + own, f"case {CASES[i]}: {err:.3e} of full scale from the chain (its own error {own:.2e})"


# Contexts whose last block is partial, one per loader: f16 group 4 and 1,
# f32 group 1 at head_dim 64 (line order) and 128, f32 group 4, and blocks
# running past the capacity.
GARBAGE_CASES = [(8, 2, 128, 65, 256, True, False), (6, 6, 64, 1499, 1500, True, True),
                 (6, 6, 64, 37, 448, False, True), (4, 4, 64, 33, 452, False, True),
                 (2, 2, 128, 330, 332, False, False), (8, 2, 128, 1001, 1002, False, False),
                 (4, 4, 64, 33, 452, True, True)]


@pytest.mark.parametrize("case", GARBAGE_CASES)
def test_positions_past_tk_never_reach_the_context(gpu, case):
    """The reference layouts' last block may read positions tk .. cap - 1:
    filled with NaN there, the context is bit-identical to the finite fill."""
    from ttsxabe_amd.gpu import DecodeScratch
    heads, kv, hd, tk, cap, half, scale_q = case
    q = oracle.seq(heads * hd, 7)
    k0 = oracle.seq(kv * cap * hd, 8).reshape(kv, cap, hd)
    v0 = oracle.seq(kv * hd * cap, 9).reshape(kv, hd, cap)
    kn, vn = k0.copy(), v0.copy()
    kn[:, tk:, :] = np.nan
    vn[:, :, tk:] = np.nan
    put = up_f16 if half else up
    f = gpu.attn_decode_f16 if half else gpu.attn_decode
    s = DecodeScratch()
    a = down(f(up(q), put(k0.ravel()), put(v0.ravel()), heads, kv, hd, tk, cap, 0.11, scale_q, s))
    b = down(f(up(q), put(kn.ravel()), put(vn.ravel()), heads, kv, hd, tk, cap, 0.11, scale_q, s))
    assert np.isfinite(b).all() and np.array_equal(a, b)


def test_decode_refusals(gpu):
    from ttsxabe_amd.gpu import DecodeScratch, UnsupportedAttention, CacheOverrun
    s = DecodeScratch()
    dq = up(oracle.seq(8 * 128, 1))
    dk = up_f16(oracle.seq(2 * 256 * 128, 2))
    with pytest.raises(UnsupportedAttention):
        gpu.attn_decode_f16(dq, dk, dk, 8, 2, 96, 10, 256, 1.0, False, s)
    with pytest.raises(CacheOverrun):
        gpu.attn_decode_f16(dq, dk, dk, 8, 2, 128, 257, 256, 1.0, False, s)
    with pytest.raises(CacheOverrun):
        gpu.attn_decode_f16(dq, dk, dk, 8, 2, 128, 0, 256, 1.0, False, s)
    big = up(oracle.seq(34 * 128, 1))
    with pytest.raises(UnsupportedAttention):  # a group wider than the 16 the MFMA tile carries
        gpu.attn_decode_f16(big, dk, dk, 34, 2, 128, 10, 256, 1.0, False, s)


@pytest.mark.parametrize("shape", [(8, 2, 128, 40, 64), (8, 2, 128, 1000, 1024), (4, 4, 64, 300, 512)])
def test_the_decode_attention_twin_is_the_quantiser_over_its_output(gpu, shape):
    from ttsxabe_amd.gpu import DecodeScratch
    heads, kv, hd, tk, cap = shape
    s = DecodeScratch()
    dq = up(oracle.seq(heads * hd, 61))
    dk = up_f16(oracle.seq(kv * cap * hd, 62))
    dv = up_f16(oracle.seq(kv * cap * hd, 63))
    scale = hd ** -0.5
    plain = down(gpu.attn_decode_f16(dq, dk, dv, heads, kv, hd, tk, cap, scale, True, s))
    out, twin = gpu.attn_decode_f16_q(dq, dk, dv, heads, kv, hd, tk, cap, scale, True, s)
    out = down(out)
    assert np.array_equal(plain, out), "the context differs with the twin asked for"
    wc, ws = oracle.twin_quantize(out)
    gc, gs = twin.parts()
    assert np.array_equal(wc, gc.numpy()), "codes"
    assert np.array_equal(ws, gs.numpy()), "scales"


def test_the_decode_attention_into_a_row_is_the_decode_attention(gpu):
    from ttsxabe_amd.gpu import DecodeScratch, MismatchedQ8, SliceOverrun
    heads, kv, hd, tk, cap = 8, 8, 128, 37, 64
    n = heads * hd
    rows = 3
    qs = oracle.seq(rows * n, 81)
    dk = up_f16(oracle.seq(kv * cap * hd, 82))
    dv = up_f16(oracle.seq(kv * cap * hd, 83))
    s = DecodeScratch()
    row = 1
    want, want_q = gpu.attn_decode_f16_q(up(qs[row * n:(row + 1) * n]), dk, dv, heads, kv, hd, tk, cap, 0.1, False, s)
    want = down(want)
    wc, ws = want_q.parts()
    before = oracle.seq(rows * n, 84)
    out = up(before)
    twin = gpu.q8_zeros(rows, n)
    gpu.attn_decode_f16_q_row(up(qs), row * n, dk, dv, heads, kv, hd, tk, cap, 0.1, False, s, out, twin, row)
    got = down(out)
    assert np.array_equal(got[row * n:(row + 1) * n], want)
    assert np.array_equal(got[:row * n], before[:row * n])
    assert np.array_equal(got[(row + 1) * n:], before[(row + 1) * n:])
    gc, gs = twin.parts()
    assert np.array_equal(gc[row * n:(row + 1) * n].numpy(), wc.numpy())
    assert np.array_equal(gs[row * n // 32:(row + 1) * n // 32].numpy(), ws.numpy())
    assert (gc[:row * n] == 0).all()
    with pytest.raises((MismatchedQ8, SliceOverrun)):
        gpu.attn_decode_f16_q_row(up(qs), row * n, dk, dv, heads, kv, hd, tk, cap, 0.1, False, s, out, twin, rows)
    short = gpu.q8_zeros(1, n)
    with pytest.raises(MismatchedQ8):
        gpu.attn_decode_f16_q_row(up(qs), row * n, dk, dv, heads, kv, hd, tk, cap, 0.1, False, s, out, short, row)


def test_one_scratch_serves_alternating_inputs(gpu):
    """Partials handed between workgroups must never be read stale: two
    different queries and caches alternate through one scratch, each call
    checked against the chain (a stale partial would carry the other call's
    numbers, which a same-input repeat cannot show)."""
    from ttsxabe_amd.gpu import DecodeScratch
    heads, kv, hd, tk, cap = 32, 8, 128, 4096, 4096
    s = DecodeScratch()
    cases = []
    for salt in (700, 710):
        q = oracle.seq(heads * hd, salt)
        k = oracle.through_f16(oracle.seq(kv * cap * hd, salt + 1))
        v = oracle.through_f16(oracle.seq(kv * hd * cap, salt + 2))
        exact = oracle.decode_f64(q, k, v, heads, kv, hd, tk, cap, 0.11)
        cases.append((up(q), up_f16(k), up_f16(v), exact))
    for rep in range(6):
        q, k, v, exact = cases[rep % 2]
        got = down(gpu.attn_decode_f16(q, k, v, heads, kv, hd, tk, cap, 0.11, False, s))
        assert full_scale_err(exact, got) < 2e-5, f"call {rep}"
