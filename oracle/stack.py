"""CPU restatement of a Llama decoder stack -- TEST INFRASTRUCTURE ONLY.

The arithmetic of the reference's chat model, step by step, in numpy f32 on
the CPU, for the random-init argmax check of the GPU stack
(ttsxabe_amd/stack.py). Only tests/ import it.

Follows:
  rms_norm     crates/llmtie-dsp/src/rope.rs:16-28 (mean of squares in f32,
               1/sqrt(mean + eps), times the weight; no mean subtraction)
  silu_mul     crates/llmtie-dsp/src/rope.rs:43-48 (a * 1/(1+e^-a) * b)
  linear       crates/llmtie-dsp/src/linear.rs:12-33 (x @ w.T, w [out, in])
  rope         oracle.rope = crates/llmtie-dsp/src/rope.rs:83-126
  layer order  crates/llmtie-chat/src/model.rs:700-1175: h += attn(norm(h));
               h += ffn(norm(h)); logits = lm_head(norm(h)); K/V are held in
               the cache at f16 (rope_cache_f16 / cache_append_f16 round to
               nearest even), attention is the f32 softmax of
               crates/llmtie-cuda/tests/kernels.rs:2733-2780 per query row,
               causal over past + r.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import rope as _rope
from . import through_f16


@dataclass(frozen=True)
class StackConfig:
    vocab: int = 512
    hidden: int = 512
    heads: int = 8
    kv_heads: int = 2
    head_dim: int = 64
    ffn: int = 1024
    layers: int = 2
    theta: float = 500000.0
    eps: float = 1e-5


def random_weights(cfg: StackConfig, seed: int) -> dict:
    """Seeded f32 weights, scaled so activations stay O(1) through the stack."""
    rng = np.random.default_rng(seed)
    h, kvd, f = cfg.hidden, cfg.kv_heads * cfg.head_dim, cfg.ffn

    def mat(o, i):
        return (rng.standard_normal((o, i)) / np.sqrt(i)).astype(np.float32)

    w = {"embed": rng.standard_normal((cfg.vocab, h)).astype(np.float32),
         "norm": (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32),
         "lm_head": mat(cfg.vocab, h)}
    for l in range(cfg.layers):
        w[f"{l}.attn_norm"] = (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32)
        w[f"{l}.ffn_norm"] = (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32)
        w[f"{l}.wq"] = mat(cfg.heads * cfg.head_dim, h)
        w[f"{l}.wk"] = mat(kvd, h)
        w[f"{l}.wv"] = mat(kvd, h)
        w[f"{l}.wo"] = mat(h, cfg.heads * cfg.head_dim)
        w[f"{l}.wg"] = mat(f, h)
        w[f"{l}.wu"] = mat(f, h)
        w[f"{l}.wd"] = mat(h, f)
    return w


def rms_norm(x, weight, eps):
    """rope.rs:16-28, per row."""
    x = np.asarray(x, np.float32)
    ms = (x * x).sum(axis=-1, dtype=np.float32, keepdims=True) / np.float32(x.shape[-1])
    scale = np.float32(1.0) / np.sqrt(ms + np.float32(eps))
    return (x * scale * weight).astype(np.float32)


def silu_mul(a, b):
    """rope.rs:43-48."""
    a = np.asarray(a, np.float32)
    return (a * (np.float32(1.0) / (np.float32(1.0) + np.exp(-a))) * b).astype(np.float32)


def linear(x, w):
    """linear.rs:12-33 without bias."""
    return (np.asarray(x, np.float32) @ np.asarray(w, np.float32).T).astype(np.float32)


def attend(q, kc, vc, past, n, heads, kv_heads, hd, scale):
    """Causal f32 attention of n query rows (positions past..past+n-1) over
    the f16-valued caches kc, vc [kv][pos][hd]."""
    group = heads // kv_heads
    out = np.empty((n, heads * hd), np.float32)
    qh = q.reshape(n, heads, hd)
    for r in range(n):
        tk = past + r + 1
        for h in range(heads):
            kh = h // group
            s = (kc[kh, :tk] @ qh[r, h]).astype(np.float32) * np.float32(scale)
            p = np.exp(s - s.max()).astype(np.float32)
            out[r, h * hd:(h + 1) * hd] = (p @ vc[kh, :tk]) / p.sum(dtype=np.float32)
    return out


class CpuStack:
    """The stack's forward on the CPU with its own K/V cache."""

    def __init__(self, cfg: StackConfig, w: dict):
        self.cfg, self.w = cfg, w
        self.k = [np.zeros((cfg.kv_heads, 0, cfg.head_dim), np.float32) for _ in range(cfg.layers)]
        self.v = [np.zeros((cfg.kv_heads, 0, cfg.head_dim), np.float32) for _ in range(cfg.layers)]

    @property
    def past(self) -> int:
        return self.k[0].shape[1]

    def forward(self, ids) -> np.ndarray:
        """Logits [vocab] of the last of `ids`, appended after the cache."""
        c, w = self.cfg, self.w
        n, past, hd = len(ids), self.past, c.head_dim
        h = w["embed"][np.asarray(ids)].astype(np.float32)
        for l in range(c.layers):
            x = rms_norm(h, w[f"{l}.attn_norm"], c.eps)
            q = linear(x, w[f"{l}.wq"])
            k = linear(x, w[f"{l}.wk"])
            v = linear(x, w[f"{l}.wv"])
            fd = w.get("rope_freqs")  # Llama-3 per-frequency divisors (rope.rs:83-126), if bound
            q = _rope(q, n, c.heads, hd, c.theta, past, fd).reshape(n, -1)
            k = _rope(k, n, c.kv_heads, hd, c.theta, past, fd).reshape(n, -1)
            kk = through_f16(k).reshape(n, c.kv_heads, hd).transpose(1, 0, 2)
            vv = through_f16(v).reshape(n, c.kv_heads, hd).transpose(1, 0, 2)
            self.k[l] = np.concatenate([self.k[l], kk], axis=1)
            self.v[l] = np.concatenate([self.v[l], vv], axis=1)
            ctx = attend(q, self.k[l], self.v[l], past, n, c.heads, c.kv_heads, hd, np.float32(hd) ** np.float32(-0.5))
            h = h + linear(ctx, w[f"{l}.wo"])
            x = rms_norm(h, w[f"{l}.ffn_norm"], c.eps)
            h = h + linear(silu_mul(linear(x, w[f"{l}.wg"]), linear(x, w[f"{l}.wu"])), w[f"{l}.wd"])
        return linear(rms_norm(h[-1:], w["norm"], c.eps), w["lm_head"])[0]
