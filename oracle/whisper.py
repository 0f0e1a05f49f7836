"""CPU restatement of the Whisper cross-attention cache build -- TEST
INFRASTRUCTURE ONLY (only tests/ import it).

crates/llmtie-asr/src/model.rs:871-955: the encoder output narrowed to f16,
per layer K = x16 @ Wk16.T and V = x16 @ Wv16.T + b accumulated wide and
rounded once to f16 (nearest even) into K [heads][t][hd] and
V^T [heads][hd][t]. Accumulated here in f64 and rounded to f32 before the f16
rounding, which is what an f32-accumulating GEMM approximates.
"""
from __future__ import annotations

import numpy as np

from . import f32_to_f16


def cross_cache_ref(enc, wk, wv, bv, heads):
    """enc [t, d] f32; wk, wv [layers, d, d] ([out, in]); bv [layers, d].
    Returns per layer (K bits [heads, t, hd], V bits [heads, hd, t]) as uint16."""
    enc = np.asarray(enc, np.float32)
    t, d = enc.shape
    hd = d // heads
    x = enc.astype(np.float16).astype(np.float64)
    out = []
    for l in range(wk.shape[0]):
        k = (x @ np.asarray(wk[l], np.float16).astype(np.float64).T).astype(np.float32)
        v = (x @ np.asarray(wv[l], np.float16).astype(np.float64).T).astype(np.float32) + np.asarray(bv[l], np.float32)
        kb = f32_to_f16(k).reshape(t, heads, hd).transpose(1, 0, 2)
        vb = f32_to_f16(v).reshape(t, heads, hd).transpose(1, 2, 0)
        out.append((np.ascontiguousarray(kb), np.ascontiguousarray(vb)))
    return out
