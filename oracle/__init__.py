"""CPU oracle for the attention hot path -- TEST INFRASTRUCTURE ONLY.

numpy-facing wrappers over oracle/liboracle.so (the C restatement of the
reference's scalar arithmetic in oracle.c, each function citing the reference
file:line it follows). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this package, and only as the checker or the timed
CPU baseline; the product (ttsxabe_amd) never does.

Pinning status of each function (see tests/test_oracle.py):
  f32_to_f16 / f16_to_f32   pinned: numpy float16 (IEEE RNE) on all 2^16 halves
                            and on edge/tie/subnormal f32 inputs
  seq                       pinned: reference's own xorshift recurrence run in
                            Python big ints (tests/golden); range [-2, 6)
  normal                    pinned: moments and KS statistic (generator only)
  rope                      pinned: complex-rotation closed form in f64,
                            position 0 identity, pair-norm preservation
  decode_f64                pinned: numpy f64 closed form
  decode_ref                pinned: f64 softmax closed form (scipy), uniform
                            scores -> mean of V, one key -> V, hand case
  prefill_ref               pinned: f64 torch SDPA on f16-rounded operands,
                            causal-row independence, hand case
  prefill_f32               pinned: f64 closed form
  q8_0_dequant / quantize   pinned: GGUF block closed form, round trip error
                            <= d/2, hand case with ties
  twin_quantize             pinned: hand cases incl. half-even ties
  decode_q8_batch           pinned: equals decode_ref on the dequantised cache
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_lib = None


def lib():
    """Loads (building first if absent) the oracle shared library."""
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            from . import build as _b
            _b.build()
        _lib = C.CDLL(str(_LIB_PATH))
        _declare(_lib)
    return _lib


P = C.c_void_p
I = C.c_int
F = C.c_float
U64 = C.c_uint64
SZ = C.c_size_t


def _declare(L):
    L.orc_f32_to_f16.restype = C.c_uint16
    L.orc_f32_to_f16.argtypes = [F]
    L.orc_f16_to_f32.restype = F
    L.orc_f16_to_f32.argtypes = [C.c_uint16]
    L.orc_f32_to_f16_n.argtypes = [P, P, SZ]
    L.orc_f16_to_f32_n.argtypes = [P, P, SZ]
    L.orc_seq.argtypes = [P, SZ, U64]
    L.orc_normal.argtypes = [P, SZ, U64, U64]
    L.orc_uniform_int.argtypes = [P, SZ, U64, C.c_int32, C.c_int32]
    L.orc_rope.argtypes = [P, I, I, I, F, I, P]
    L.orc_decode_ref.argtypes = [P, P, P, I, I, I, I, I, F, I, P]
    L.orc_decode_f64.argtypes = [P, P, P, I, I, I, I, I, F, I, P]
    L.orc_decode_f16.argtypes = [P, P, P, I, I, I, I, I, F, I, P, I]
    L.orc_q8_0_dequant.argtypes = [P, P, SZ, P]
    L.orc_q8_0_quantize.argtypes = [P, SZ, P, P]
    L.orc_twin_quantize.argtypes = [P, SZ, P, P]
    L.orc_decode_q8_batch.argtypes = [P, P, P, P, P, P, P, I, I, I, I, I, F, I, P, I]
    L.orc_prefill_ref.argtypes = [P, I, P, P, I, I, I, I, I, I, F, I, I, P, P, I]
    L.orc_prefill_f32.argtypes = [P, P, P, I, I, I, I, F, I, P, I]
    L.orc_has_openmp.restype = I


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data_as(P)


# ----------------------------------------------------------------- binary16

def f32_to_f16(x) -> np.ndarray:
    """IEEE binary16 RNE bits (uint16) of f32 values."""
    x, px = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(px, out.ctypes.data_as(P), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h, ph = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_n(ph, out.ctypes.data_as(P), h.size)
    return out


def through_f16(x) -> np.ndarray:
    """f32 values rounded to f16 and back (the reference test's through_f16)."""
    return f16_to_f32(f32_to_f16(x))


# --------------------------------------------------------------- generators

def seq(n: int, salt: int) -> np.ndarray:
    """crates/llmtie-cuda/tests/kernels.rs:35-46."""
    out = np.empty(n, np.float32)
    lib().orc_seq(out.ctypes.data_as(P), n, salt)
    return out


def normal(n: int, seed: int, first: int = 0) -> np.ndarray:
    """Counter-based N(0,1) (splitmix64 + Box-Muller), element i from (seed, first+i)."""
    out = np.empty(n, np.float32)
    lib().orc_normal(out.ctypes.data_as(P), n, seed, first)
    return out


def uniform_int(n: int, seed: int, lo: int, hi: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    lib().orc_uniform_int(out.ctypes.data_as(P), n, seed, lo, hi)
    return out


# --------------------------------------------------------------------- math

def rope(x, t, heads, hd, theta, first, freq_div=None) -> np.ndarray:
    """crates/llmtie-dsp/src/rope.rs:83-126; returns a rotated copy."""
    y = np.array(x, dtype=np.float32, copy=True).ravel()
    div = None
    if freq_div is not None:
        div, pdiv = _c(freq_div, np.float32)
    lib().orc_rope(y.ctypes.data_as(P), t, heads, hd, theta, first, None if div is None else pdiv)
    return y


def decode_ref(q, k, v, heads, kv, hd, tk, cap, scale, scale_q) -> np.ndarray:
    """crates/llmtie-cuda/tests/kernels.rs:2733-2780 (f32)."""
    q, pq = _c(q, np.float32)
    k, pk = _c(k, np.float32)
    v, pv = _c(v, np.float32)
    out = np.empty(heads * hd, np.float32)
    lib().orc_decode_ref(pq, pk, pv, heads, kv, hd, tk, cap, scale, int(scale_q), out.ctypes.data_as(P))
    return out


def decode_f64(q, k, v, heads, kv, hd, tk, cap, scale, scale_q=False) -> np.ndarray:
    """decode_ref's computation in f64 (the exact value it approximates)."""
    q, pq = _c(q, np.float32)
    k, pk = _c(k, np.float32)
    v, pv = _c(v, np.float32)
    out = np.empty(heads * hd, np.float64)
    lib().orc_decode_f64(pq, pk, pv, heads, kv, hd, tk, cap, scale, int(scale_q), out.ctypes.data_as(P))
    return out


def decode_f16(q, k_bits, v_bits, heads, kv, hd, tk, cap, scale, scale_q, threads=1) -> np.ndarray:
    """decode_ref over an f16 cache given as bits (the CPU baseline form)."""
    q, pq = _c(q, np.float32)
    k, pk = _c(k_bits, np.uint16)
    v, pv = _c(v_bits, np.uint16)
    out = np.empty(heads * hd, np.float32)
    lib().orc_decode_f16(pq, pk, pv, heads, kv, hd, tk, cap, scale, int(scale_q), out.ctypes.data_as(P), threads)
    return out


def q8_0_dequant(codes, scales) -> np.ndarray:
    """crates/llmtie-gguf/src/dequant.rs:180-185."""
    codes, pc = _c(codes, np.int8)
    scales, ps = _c(scales, np.uint16)
    out = np.empty(codes.shape, np.float32)
    lib().orc_q8_0_dequant(pc, ps, codes.size, out.ctypes.data_as(P))
    return out


def q8_0_quantize(x):
    """ggml quantize_row_q8_0_ref: (codes int8, scales f16 bits)."""
    x, px = _c(x, np.float32)
    codes = np.empty(x.shape, np.int8)
    scales = np.empty(x.size // 32, np.uint16)
    lib().orc_q8_0_quantize(px, x.size, codes.ctypes.data_as(P), scales.ctypes.data_as(P))
    return codes, scales


def twin_quantize(y):
    """crates/llmtie-cuda/src/kernels.rs:5755-5773: (codes int8, scales f32)."""
    y, py = _c(y, np.float32)
    codes = np.empty(y.shape, np.int8)
    scales = np.empty(y.size // 32, np.float32)
    lib().orc_twin_quantize(py, y.size, codes.ctypes.data_as(P), scales.ctypes.data_as(P))
    return codes, scales


def decode_q8_batch(q, kc, ks, vc, vs, tk, slot, heads, kv, hd, cap, scale, scale_q, threads=1) -> np.ndarray:
    nseq = len(tk)
    q, pq = _c(q, np.float32)
    kc, pkc = _c(kc, np.int8)
    ks, pks = _c(ks, np.uint16)
    vc, pvc = _c(vc, np.int8)
    vs, pvs = _c(vs, np.uint16)
    tk, ptk = _c(tk, np.int32)
    slot, psl = _c(slot, np.int32)
    out = np.empty(nseq * heads * hd, np.float32)
    lib().orc_decode_q8_batch(pq, pkc, pks, pvc, pvs, ptk, psl, nseq, heads, kv, hd, cap, scale, int(scale_q),
                              out.ctypes.data_as(P), threads)
    return out


def prefill_ref(q, qs, k, v, tq, past, heads, kv, hd, cap, scale, causal, scale_q=False, threads=8):
    """crates/llmtie-cuda/tests/kernels.rs:2290-2374: (want f64, spread f64)."""
    q, pq = _c(q, np.float32)
    k, pk = _c(k, np.float32)
    v, pv = _c(v, np.float32)
    want = np.empty(tq * heads * hd, np.float64)
    spread = np.empty(tq * heads * hd, np.float64)
    lib().orc_prefill_ref(pq, qs, pk, pv, tq, past, heads, kv, hd, cap, scale, int(causal), int(scale_q),
                          want.ctypes.data_as(P), spread.ctypes.data_as(P), threads)
    return want, spread


def prefill_f32(q, k, v, t, heads, kv, hd, scale, causal=True, threads=1) -> np.ndarray:
    """Config-1 CPU prefill (f32 chain per row)."""
    q, pq = _c(q, np.float32)
    k, pk = _c(k, np.float32)
    v, pv = _c(v, np.float32)
    out = np.empty(t * heads * hd, np.float32)
    lib().orc_prefill_f32(pq, pk, pv, t, heads, kv, hd, scale, int(causal), out.ctypes.data_as(P), threads)
    return out


def has_openmp() -> bool:
    return bool(lib().orc_has_openmp())
