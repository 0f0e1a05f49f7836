"""The five benchmark configs C1-C5 as seeded synthetic workloads (shared by the
config parity tests, smoke() and bench.py). Inputs come from the oracle's
counter-based generators, so any rank or test regenerates them bit-exactly.
"""
from __future__ import annotations

import numpy as np

import oracle

SEED = 20261201
THETA = 500000.0


def rope_rows(x, t, heads, hd, first=0):
    return oracle.rope(x, t, heads, hd, THETA, first)


def kv_caches_f16(k_rows, v_rows, t, kv, hd, cap):
    """[t][kv*hd] f32 rows -> f16-bit caches K [kv][cap][hd], V [kv][hd][cap]."""
    kr = k_rows.reshape(t, kv, hd)
    vr = v_rows.reshape(t, kv, hd)
    kc = np.zeros((kv, cap, hd), np.float32)
    vc = np.zeros((kv, hd, cap), np.float32)
    kc[:, :t] = kr.transpose(1, 0, 2)
    vc[:, :, :t] = vr.transpose(1, 2, 0)
    return oracle.f32_to_f16(kc.ravel()), oracle.f32_to_f16(vc.ravel())


def c2_decode(seed=SEED, heads=32, kv=8, hd=128, tk=4096):
    """Llama-3-8B GQA decode: q rotated at tk-1, K rotated at 0..tk-1."""
    q = rope_rows(oracle.normal(heads * hd, seed, 0), 1, heads, hd, tk - 1)
    k = rope_rows(oracle.normal(tk * kv * hd, seed + 1), tk, kv, hd, 0)
    v = oracle.normal(tk * kv * hd, seed + 2)
    kc, vc = kv_caches_f16(k, v, tk, kv, hd, tk)
    return dict(q=q, k=kc, v=vc, heads=heads, kv=kv, hd=hd, tk=tk, cap=tk, scale=hd ** -0.5, scale_q=False)


def c3_prefill(tq, seed=SEED + 10, heads=32, kv=8, hd=128):
    """Causal GQA prefill of tq tokens from position 0, RoPE on q and k."""
    q = rope_rows(oracle.normal(tq * heads * hd, seed), tq, heads, hd, 0)
    k = rope_rows(oracle.normal(tq * kv * hd, seed + 1), tq, kv, hd, 0)
    v = oracle.normal(tq * kv * hd, seed + 2)
    kc, vc = kv_caches_f16(k, v, tq, kv, hd, tq)
    return dict(q=q, k=kc, v=vc, tq=tq, past=0, heads=heads, kv=kv, hd=hd, cap=tq, scale=hd ** -0.5)


def c4_encoder(seed=SEED + 20, t=1500, heads=20, hd=64):
    """Whisper large-v2 encoder self-attention off the stacked [t, 3d] rows."""
    return dict(qkv=oracle.normal(t * 3 * heads * hd, seed), t=t, heads=heads, hd=hd, scale=hd ** -0.5)


def c4_cross(seed=SEED + 30, heads=20, hd=64, tk=1500):
    """Whisper decoder cross-attention: one query over the 1500 encoder K/V (f16)."""
    q = oracle.normal(heads * hd, seed)
    k = oracle.normal(tk * heads * hd, seed + 1)
    v = oracle.normal(tk * heads * hd, seed + 2)
    kc, vc = kv_caches_f16(k, v, tk, heads, hd, tk)
    return dict(q=q, k=kc, v=vc, heads=heads, kv=heads, hd=hd, tk=tk, cap=tk, scale=hd ** -0.5, scale_q=True)


def c4_self(seed=SEED + 40, heads=20, hd=64, tk=224, cap=448):
    """Whisper decoder self-attention over a 224-position cache (f32, cap 448, as the reference keeps it)."""
    q = oracle.normal(heads * hd, seed)
    k = oracle.normal(tk * heads * hd, seed + 1)
    v = oracle.normal(tk * heads * hd, seed + 2)
    kc = np.zeros((heads, cap, hd), np.float32)
    vc = np.zeros((heads, hd, cap), np.float32)
    kc[:, :tk] = k.reshape(tk, heads, hd).transpose(1, 0, 2)
    vc[:, :, :tk] = v.reshape(tk, heads, hd).transpose(1, 2, 0)
    return dict(q=q, k=kc.ravel(), v=vc.ravel(), heads=heads, kv=heads, hd=hd, tk=tk, cap=cap, scale=hd ** -0.5,
                scale_q=True)


def c5_lengths(seed=SEED + 50, nseq=32):
    return oracle.uniform_int(nseq, seed, 256, 8192)


def c5_q8(seed=SEED + 50, nseq=32, heads=32, kv=8, hd=128, cap=8192, slots=None):
    """Batched Q8_0 decode: codes ~ U{-127..127}, scales ~ |N(0, 0.02)| (f16),
    lengths ~ U[256, 8192]; sequence s in slot s."""
    slots = nseq if slots is None else slots
    tk = c5_lengths(seed, nseq)
    n = slots * kv * cap * hd
    kc = oracle.uniform_int(n, seed + 1, -127, 127).astype(np.int8)
    vc = oracle.uniform_int(n, seed + 2, -127, 127).astype(np.int8)
    ks = oracle.f32_to_f16(np.abs(oracle.normal(n // 32, seed + 3)) * np.float32(0.02))
    vs = oracle.f32_to_f16(np.abs(oracle.normal(n // 32, seed + 4)) * np.float32(0.02))
    q = oracle.normal(nseq * heads * hd, seed + 5)
    return dict(q=q, kc=kc, ks=ks, vc=vc, vs=vs, tk=tk, slot=np.arange(nseq, dtype=np.int32) % slots, nseq=nseq,
                heads=heads, kv=kv, hd=hd, cap=cap, slots=slots, scale=hd ** -0.5, scale_q=False)


def c1_cpu(seed=SEED + 60, t=128, heads=8, hd=64):
    """Config 1: f32 causal MHA prefill on the CPU path."""
    return dict(q=oracle.normal(t * heads * hd, seed), k=oracle.normal(t * heads * hd, seed + 1),
                v=oracle.normal(t * heads * hd, seed + 2), t=t, heads=heads, hd=hd, scale=hd ** -0.5)
