"""The Whisper cross-attention cache build (crates/llmtie-asr/src/model.rs:
871-955) at Whisper large-v2's shape (1500 positions, d_model 1280, 20
heads) for two decoder layers: the cache this library's producers write from
the projections, in both layouts, against the CPU restatement
(oracle/whisper.py), then a cross-attention decode over it.

The GEMM accumulates in f32 on the GPU and in f64 on the CPU, so a value
sitting on an f16 rounding boundary may round one way or the other: the bar
is one f16 ulp of the value (with an absolute floor of 2^-16 for near-zero
values) and bit equality for more than 99 % of the values.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle.whisper import cross_cache_ref
from tests.configs import SEED
from tests.tiled import pack_t16, unpack_t16
from tests.util import down, full_scale_err, up

pytestmark = pytest.mark.gpu

T, D, HEADS, LAYERS = 1500, 1280, 20, 2


def _inputs():
    rng = np.random.default_rng(SEED + 7)
    enc = rng.standard_normal((T, D)).astype(np.float32)
    wk = (rng.standard_normal((LAYERS, D, D)) / np.sqrt(D)).astype(np.float32)
    wv = (rng.standard_normal((LAYERS, D, D)) / np.sqrt(D)).astype(np.float32)
    bv = (0.1 * rng.standard_normal((LAYERS, D))).astype(np.float32)
    return enc, wk, wv, bv


@pytest.mark.parametrize("layout", ["reference", "tiled"])
def test_cross_cache_build_matches_cpu_and_decodes(gpu, layout):
    from ttsxabe_amd.gpu import DecodeScratch
    from ttsxabe_amd.whisper import build_cross_cache
    enc, wk, wv, bv = _inputs()
    want = cross_cache_ref(enc, wk, wv, bv, HEADS)
    got = build_cross_cache(gpu, up(enc), up(wk), up(wv), up(bv), HEADS, layout)
    hd = D // HEADS
    for l in range(LAYERS):
        if layout == "tiled":
            # the tiled cache against the CPU cache packed by the numpy packer
            pairs = (("K+V tiled", down(got[l].data).view(np.uint16),
                      pack_t16(want[l][0], want[l][1], HEADS, hd, T)),)
        else:
            pairs = (("K", down(got[l][0]).view(np.uint16).reshape(HEADS, T, hd), want[l][0]),
                     ("V", down(got[l][1]).view(np.uint16).reshape(HEADS, hd, T), want[l][1]))
        for name, g, w in pairs:
            gv = g.view(np.float16).astype(np.float64)
            wv_ = w.view(np.float16).astype(np.float64)
            # one f16 ulp of the value, or an absolute 2^-16 for near-zero
            # values: the f32 GEMM's own error against f64 measures up to
            # ~8e-6 on these O(1) products, many ulps of a tiny result
            big = np.maximum(np.abs(gv), np.abs(wv_)).astype(np.float16)
            tol = np.maximum(np.spacing(big).astype(np.float64), 2.0 ** -16)
            bad = np.abs(gv - wv_) > tol
            eq = (g == w).mean()
            idx = np.flatnonzero(bad.ravel())[:3].tolist() + [int(np.abs(gv - wv_).argmax())]
            assert not bad.any(), (f"layer {l} {name}: {int(bad.sum())} beyond tolerance, worst "
                                   f"{np.abs(gv - wv_).max():.3g}; e.g. at {idx} got "
                                   f"{gv.ravel()[idx].tolist()} want {wv_.ravel()[idx].tolist()}")
            # a GEMM error of ~2e-6 relative flips the f16 rounding of the
            # ~0.4 % of values that lie that close to a rounding boundary
            assert eq > 0.99, f"layer {l} {name}: only {eq:.5f} bit-equal"
    # a cross-attention step over the last layer's cache (scale on the query)
    q = oracle.seq(HEADS * hd, 901)
    scale = float(np.float32(hd) ** np.float32(-0.5))
    # parity of the decode on the cache it reads (the GPU-built one)
    if layout == "tiled":
        kb, vb = unpack_t16(down(got[-1].data).view(np.uint16), HEADS, hd, T)
    else:
        kb, vb = down(got[-1][0]).view(np.uint16), down(got[-1][1]).view(np.uint16)
    kf, vf = oracle.f16_to_f32(kb), oracle.f16_to_f32(vb)
    exact = oracle.decode_f64(q, kf, vf, HEADS, HEADS, hd, T, T, scale, True)
    s = DecodeScratch()
    if layout == "tiled":
        out = gpu.attn_decode_t16(up(q), got[-1], HEADS, T, scale, True, s)
    else:
        out = gpu.attn_decode_f16(up(q), got[-1][0], got[-1][1], HEADS, HEADS, hd, T, T, scale, True, s)
    assert full_scale_err(exact, down(out)) < 2e-5
