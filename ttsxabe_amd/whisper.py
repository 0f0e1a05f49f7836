"""The Whisper decoder's cross-attention cache, built from the encoder output.

crates/llmtie-asr/src/model.rs:871-955 (`Model::cache`): the encoder output
[t, d] is narrowed to f16 once; every decoder layer's key and value
projections of it run as one batched f16 GEMM with f32 accumulation (plain
torch here: a library GEMM is plumbing); the f32 products are split into the
f16 cache layouts the cross-attention decode reads -- K [heads][t][hd] and
V^T [heads][hd][t], rounded to nearest even, the value bias added in f32
before the rounding -- or into the tiled fragment-order cache. The split goes
through this library's cache producers (cache_append_f16 / t16_append with
n = t, past = 0, cap = t), so the layout logic under test is the product's.
"""
from __future__ import annotations

import torch

from .gpu import Gpu, TiledCache16


def cross_projections(encoded: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """[layers, t, d] f32 = f16(encoded) @ f16(w[l]).T for every layer l.
    f16 operands are exact in f32 and their products are exact, so f32
    matmul of the narrowed operands is the f16 GEMM with f32 accumulation."""
    narrow = encoded.to(torch.float16).to(torch.float32)
    return torch.matmul(narrow.unsqueeze(0), w.to(torch.float16).to(torch.float32).transpose(1, 2))


def build_cross_cache(g: Gpu, encoded: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor, bv: torch.Tensor,
                      heads: int, layout: str = "reference"):
    """encoded [t, d] f32; wk, wv [layers, d, d] (f16 or f32, `nn.Linear`
    layout [out, in]); bv [layers, d] f32. Returns per layer (K, V) f16
    tensors in the reference layout, or a TiledCache16 per layer."""
    t, d = encoded.shape
    layers = wk.shape[0]
    hd = d // heads
    if hd * heads != d:
        raise ValueError(f"d_model {d} is not heads {heads} x head_dim")
    k_all = cross_projections(encoded, wk)
    out = []
    for i in range(layers):
        k = k_all[i].contiguous().view(-1)
        if layout == "tiled":
            c = TiledCache16(heads, hd, t, device=g.device)
            g.t16_append(k, 0, c, t, 0, False)
            out.append(c)
        else:
            kc = torch.empty(t * d, dtype=torch.float16, device=g.device)
            g.cache_append_f16(k, 0, kc, t, heads, hd, t, 0, False)
            out.append([kc, None])
    del k_all
    v_all = cross_projections(encoded, wv)
    for i in range(layers):
        v = (v_all[i] + bv[i]).contiguous().view(-1)
        if layout == "tiled":
            g.t16_append(v, 0, out[i], t, 0, True)
        else:
            vc = torch.empty(t * d, dtype=torch.float16, device=g.device)
            g.cache_append_f16(v, 0, vc, t, heads, hd, t, 0, True)
            out[i][1] = vc
    return out if layout == "tiled" else [tuple(p) for p in out]
