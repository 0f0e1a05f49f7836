"""The benchmark configs C1-C5 at full size against the oracle, at the north
star's bar: max |err| <= 5e-3 and per-head cosine >= 0.9999 (tolerances
written here), plus the reference's own per-element prefill rule where the
f64 reference applies.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import configs
from tests.util import down, per_head_cos, up

pytestmark = pytest.mark.gpu

MAX_ABS = 5e-3
MIN_COS = 0.9999


def check(want, got, rows, heads, hd, what):
    want = np.asarray(want, np.float64)
    got = np.asarray(got, np.float64)
    err = float(np.abs(want - got).max())
    cos = per_head_cos(want, got, rows, heads, hd)
    print(f"{what}: max abs {err:.3e}, min head cosine {cos.min():.7f}", flush=True)
    assert err <= MAX_ABS, f"{what}: max abs {err}"
    assert cos.min() >= MIN_COS, f"{what}: head cosine {cos.min()}"


def test_c1_f32_causal_mha_prefill(gpu):
    """Config 1 (f32 causal MHA, 8/8/64, 128 tokens, no RoPE) through the HIP
    f32-cache prefill, against the reference's CPU f32 chain at the north
    star's bar, and against the reference's f64 prefill rule
    (kernels.rs:2290-2374)."""
    c = configs.c1_cpu()
    t, heads, hd = c["t"], c["heads"], c["hd"]
    cpu = oracle.prefill_f32(c["q"], c["k"], c["v"], t, heads, heads, hd, c["scale"], True)
    kc = np.ascontiguousarray(c["k"].reshape(t, heads, hd).transpose(1, 0, 2)).ravel()  # [kv][cap][hd]
    vc = np.ascontiguousarray(c["v"].reshape(t, heads, hd).transpose(1, 2, 0)).ravel()  # [kv][hd][cap]
    got = down(gpu.flash_attn(up(c["q"]), up(kc), up(vc), t, 0, heads, heads, hd, t, c["scale"], True))
    check(cpu, got, t, heads, hd, "C1 f32 prefill vs the CPU f32 chain")
    want, spread = oracle.prefill_ref(c["q"], heads * hd, kc, vc, t, 0, heads, heads, hd, t, c["scale"], True)
    tol = 2e-4 + 1e-2 * np.abs(want) + 1e-2 * spread
    err = np.abs(want - got.astype(np.float64))
    assert (err <= tol).all() and float((err / tol).max()) < 0.5


def test_c2_llama3_gqa_decode(gpu):
    from ttsxabe_amd.gpu import DecodeScratch
    c = configs.c2_decode()
    k = oracle.f16_to_f32(c["k"])
    v = oracle.f16_to_f32(c["v"])
    want = oracle.decode_ref(c["q"], k, v, c["heads"], c["kv"], c["hd"], c["tk"], c["cap"], c["scale"], False)
    dk = torch.from_numpy(c["k"].view(np.float16)).cuda()
    dv = torch.from_numpy(c["v"].view(np.float16)).cuda()
    got = down(gpu.attn_decode_f16(up(c["q"]), dk, dv, c["heads"], c["kv"], c["hd"], c["tk"], c["cap"], c["scale"],
                                   False, DecodeScratch()))
    check(want, got, 1, c["heads"], c["hd"], "C2 decode")
    from ttsxabe_amd.gpu import TiledCache16
    t = TiledCache16(c["kv"], c["hd"], c["cap"])
    gpu.t16_from_ref(dk, dv, t, c["tk"])
    got_t = down(gpu.attn_decode_t16(up(c["q"]), t, c["heads"], c["tk"], c["scale"], False, DecodeScratch()))
    check(want, got_t, 1, c["heads"], c["hd"], "C2 decode (tiled cache)")


@pytest.mark.parametrize("tq", [128, 512])
def test_c3_llama3_gqa_prefill(gpu, tq):
    c = configs.c3_prefill(tq)
    k = oracle.f16_to_f32(c["k"])
    v = oracle.f16_to_f32(c["v"])
    dk = torch.from_numpy(c["k"].view(np.float16)).cuda()
    dv = torch.from_numpy(c["v"].view(np.float16)).cuda()
    got = down(gpu.flash_attn_f16(up(c["q"]), dk, dv, tq, 0, c["heads"], c["kv"], c["hd"], c["cap"], c["scale"],
                                  True)).astype(np.float64)
    want, spread = oracle.prefill_ref(c["q"], c["heads"] * c["hd"], k, v, tq, 0, c["heads"], c["kv"], c["hd"],
                                      c["cap"], c["scale"], True, threads=16)
    tol = 2e-4 + 1e-2 * np.abs(want) + 1e-2 * spread
    assert (np.abs(want - got) <= tol).all()
    check(want, got, tq, c["heads"], c["hd"], f"C3 prefill {tq}")
    from ttsxabe_amd.gpu import TiledCache16
    t = TiledCache16(c["kv"], c["hd"], c["cap"])
    gpu.t16_from_ref(dk, dv, t, tq)
    got_t = down(gpu.flash_attn_t16(up(c["q"]), t, tq, 0, c["heads"], c["scale"], True)).astype(np.float64)
    assert np.array_equal(got, got_t), "tiled-cache prefill differs from the reference-layout one"


def test_c4_whisper_encoder(gpu):
    c = configs.c4_encoder()
    t, heads, hd = c["t"], c["heads"], c["hd"]
    d = heads * hd
    rows = c["qkv"].reshape(t, 3 * d)
    q = np.ascontiguousarray(rows[:, :d])
    k = np.ascontiguousarray(rows[:, d:2 * d].reshape(t, heads, hd).transpose(1, 0, 2)).ravel()
    v = np.ascontiguousarray(rows[:, 2 * d:].reshape(t, heads, hd).transpose(1, 2, 0)).ravel()
    want, spread = oracle.prefill_ref(q, d, k, v, t, 0, heads, heads, hd, t, c["scale"], False, scale_q=True,
                                      threads=16)
    got = down(gpu.flash_attn_rows(up(c["qkv"]), t, heads, hd, c["scale"]).float()).astype(np.float64)
    # The context is f16: the rule gains the half-ulp of the output rounding.
    tol = 2e-4 + 1e-2 * np.abs(want) + 1e-2 * spread + np.abs(want) * 2.0 ** -11
    assert (np.abs(want - got) <= tol).all()
    check(want, got, t, heads, hd, "C4 encoder")


def test_c4_whisper_cross_and_self_decode(gpu):
    from ttsxabe_amd.gpu import DecodeScratch
    s = DecodeScratch()
    c = configs.c4_cross()
    want = oracle.decode_ref(c["q"], oracle.f16_to_f32(c["k"]), oracle.f16_to_f32(c["v"]), c["heads"], c["kv"],
                             c["hd"], c["tk"], c["cap"], c["scale"], True)
    dk = torch.from_numpy(c["k"].view(np.float16)).cuda()
    dv = torch.from_numpy(c["v"].view(np.float16)).cuda()
    got = down(gpu.attn_decode_f16(up(c["q"]), dk, dv, c["heads"], c["kv"], c["hd"], c["tk"], c["cap"], c["scale"],
                                   True, s))
    check(want, got, 1, c["heads"], c["hd"], "C4 cross")
    c = configs.c4_self()
    want = oracle.decode_ref(c["q"], c["k"], c["v"], c["heads"], c["kv"], c["hd"], c["tk"], c["cap"], c["scale"], True)
    got = down(gpu.attn_decode(up(c["q"]), up(c["k"]), up(c["v"]), c["heads"], c["kv"], c["hd"], c["tk"], c["cap"],
                               c["scale"], True, s))
    check(want, got, 1, c["heads"], c["hd"], "C4 self")


def test_c5_batched_q8_decode(gpu):
    from ttsxabe_amd.gpu import DecodeScratch, KvCacheQ8
    c = configs.c5_q8()
    from tests import tiled
    cache = KvCacheQ8(c["slots"], c["kv"], c["hd"], c["cap"])
    cache.data.copy_(torch.from_numpy(tiled.pack_q8(c["kc"], c["ks"], c["vc"], c["vs"], c["slots"], c["kv"], c["hd"],
                                                    c["cap"])))
    got = down(gpu.attn_decode_q8_batch(up(c["q"]), cache, up(c["tk"], torch.int32), up(c["slot"], torch.int32),
                                        c["cap"], c["heads"], c["scale"], False, DecodeScratch()))
    want = oracle.decode_q8_batch(c["q"], c["kc"], c["ks"], c["vc"], c["vs"], c["tk"], c["slot"], c["heads"],
                                  c["kv"], c["hd"], c["cap"], c["scale"], False, threads=16)
    check(want, got, c["nseq"], c["heads"], c["hd"], "C5 Q8_0 batch")
