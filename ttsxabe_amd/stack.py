"""A Llama decoder stack around the attention path, on one MI355X.

The caller side of the path as the reference's chat model arranges it
(crates/llmtie-chat/src/model.rs:700-1175): per layer RMSNorm, the q/k/v
projections, RoPE with the K/V cache write, attention, the output projection
and residual, then RMSNorm and the SwiGLU feed-forward; a final RMSNorm and
the LM head. The projections, norms and SwiGLU are plain torch f32 ops here
(plumbing); RoPE, the cache writes, cache growth and attention go through this
library, which is the part under test. Weights come from the caller (random,
for the argmax check against the CPU restatement of the same stack).

The cache grows like the reference's: to the next power of two of what is
needed, at least 256 positions (model.rs:703-721), copying the live prefix.
"""
from __future__ import annotations

import numpy as np
import torch

from .gpu import DecodeScratch, Gpu, TiledCache16


class LlamaStack:
    """`layout`: "reference" (K [kv][cap][hd] + V [kv][hd][cap] f16, the
    reference's cache) or "tiled" (the fragment-order cache)."""

    def __init__(self, gpu: Gpu, cfg, weights: dict, layout: str = "reference"):
        if layout not in ("reference", "tiled"):
            raise ValueError(f"unknown cache layout {layout!r}")
        self.g, self.cfg, self.layout = gpu, cfg, layout
        dev = gpu.device
        self.w = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in weights.items()}
        self.past = 0
        self.cap = 0
        self.kc, self.vc, self.tc = [], [], []
        self.scratch = DecodeScratch()

    def _grow(self, need: int):
        if need <= self.cap:
            return
        c = self.cfg
        want = max(256, 1 << (need - 1).bit_length())
        kvd = c.kv_heads * c.head_dim
        for l in range(c.layers):
            if self.layout == "tiled":
                t = TiledCache16(c.kv_heads, c.head_dim, want, device=self.g.device)
                if self.past:
                    self.g.t16_grow(self.tc[l], t, self.past)
                if l < len(self.tc):
                    self.tc[l] = t
                else:
                    self.tc.append(t)
            else:
                k = torch.zeros(want * kvd, dtype=torch.float16, device=self.g.device)
                v = torch.zeros(want * kvd, dtype=torch.float16, device=self.g.device)
                if self.past:
                    self.g.cache_grow_f16(self.kc[l], k, c.kv_heads, c.head_dim, self.cap, want, self.past, False)
                    self.g.cache_grow_f16(self.vc[l], v, c.kv_heads, c.head_dim, self.cap, want, self.past, True)
                if l < len(self.kc):
                    self.kc[l], self.vc[l] = k, v
                else:
                    self.kc.append(k)
                    self.vc.append(v)
        self.cap = want

    def _norm(self, x, w):
        """crates/llmtie-dsp/src/rope.rs:16-28."""
        return x * torch.rsqrt((x * x).mean(dim=-1, keepdim=True) + self.cfg.eps) * w

    def forward(self, ids) -> torch.Tensor:
        """Logits [vocab] of the last of `ids`, which extend the cache."""
        c, g, w = self.cfg, self.g, self.w
        n, past, hd = len(ids), self.past, c.head_dim
        self._grow(past + n)
        scale = float(np.float32(hd) ** np.float32(-0.5))
        fd = w.get("rope_freqs")  # Llama-3 per-frequency RoPE divisors, when the checkpoint has them
        h = w["embed"][torch.as_tensor(list(ids), device=g.device)]
        for l in range(c.layers):
            x = self._norm(h, w[f"{l}.attn_norm"])
            q = (x @ w[f"{l}.wq"].T).contiguous().view(-1)
            k = (x @ w[f"{l}.wk"].T).contiguous().view(-1)
            v = (x @ w[f"{l}.wv"].T).contiguous().view(-1)
            if self.layout == "tiled":
                t = self.tc[l]
                if n == 1:
                    g.t16_rope_cache(q, 0, k, 0, v, 0, fd, c.heads, c.theta, past, t)
                    ctx = g.attn_decode_t16(q, t, c.heads, past + 1, scale, False, self.scratch)
                else:
                    g.rope_scaled(q, 0, fd, n, c.heads, hd, c.theta, past)
                    g.rope_scaled(k, 0, fd, n, c.kv_heads, hd, c.theta, past)
                    g.t16_append(k, 0, t, n, past, False)
                    g.t16_append(v, 0, t, n, past, True)
                    ctx = g.flash_attn_t16(q, t, n, past, c.heads, scale, True)
            else:
                kc, vc = self.kc[l], self.vc[l]
                if n == 1:
                    g.rope_cache_f16(q, 0, k, 0, v, 0, fd, c.heads, c.kv_heads, hd, c.theta, past, kc, vc,
                                     self.cap)
                    ctx = g.attn_decode_f16(q, kc, vc, c.heads, c.kv_heads, hd, past + 1, self.cap, scale, False,
                                            self.scratch)
                else:
                    g.rope_scaled(q, 0, fd, n, c.heads, hd, c.theta, past)
                    g.rope_scaled(k, 0, fd, n, c.kv_heads, hd, c.theta, past)
                    g.cache_append_f16(k, 0, kc, n, c.kv_heads, hd, self.cap, past, False)
                    g.cache_append_f16(v, 0, vc, n, c.kv_heads, hd, self.cap, past, True)
                    ctx = g.flash_attn_f16(q, kc, vc, n, past, c.heads, c.kv_heads, hd, self.cap, scale, True)
            h = h + ctx.view(n, -1) @ w[f"{l}.wo"].T
            x = self._norm(h, w[f"{l}.ffn_norm"])
            h = h + (torch.nn.functional.silu(x @ w[f"{l}.wg"].T) * (x @ w[f"{l}.wu"].T)) @ w[f"{l}.wd"].T
        self.past += n
        return (self._norm(h[-1:], w["norm"]) @ w["lm_head"].T)[0]
