"""A Llama checkpoint in a GGUF, bound to the layer stack's weights.

The reference's GGUF path for its chat model: the geometry from the metadata
store (crates/llmtie-llama/src/config.rs:84-140, `LlamaConfig::from_gguf`),
every tensor bound by name and checked against that geometry
(src/weights.rs:165-230, `LlamaWeights::from_gguf`), and llama.cpp's rope
permutation of `attn_q` / `attn_k` undone at load (src/gguf.rs:32-56,
`unpermute_rope`) so that the halves rotation of this library's RoPE applies
to the loaded weights as it does to a safetensors checkpoint's.

The permutation: llama.cpp's converter reorders the rows of `attn_q` and
`attn_k` within each head so that an interleaved rotation (pairs 2i, 2i+1)
over the permuted rows equals the halves rotation (pairs i, i + hd/2) over
the original ones: original row k * hd/2 + i of a head is stored at row
2i + k. `attn_q` is divided into the query heads, `attn_k` into the kv heads.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .gguf import GgufFile


class LlamaGgufError(ValueError):
    """The GGUF is not a Llama this stack can bind (missing metadata, another
    architecture, or a tensor of the wrong shape)."""


@dataclass(frozen=True)
class LlamaConfig:
    """The stack's geometry (the fields `ttsxabe_amd.stack.LlamaStack` reads)."""
    vocab: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    layers: int
    theta: float
    eps: float


def config_from_gguf(f: GgufFile) -> LlamaConfig:
    """config.rs:84-140: `general.architecture` must be "llama"; the vocabulary
    is `llama.vocab_size`, else the tokenizer's token array; the head width
    is `llama.attention.key_length`, else hidden / heads."""
    arch = f.get_str("general.architecture")
    if arch is None:
        raise LlamaGgufError("missing metadata `general.architecture`")
    if arch != "llama":
        raise LlamaGgufError(f"architecture `{arch}`, wanted `llama`")

    def need(key):
        v = f.get_u32(key)
        if v is None:
            raise LlamaGgufError(f"missing metadata `{key}`")
        return v

    def need_f(key):
        v = f.get_f32(key)
        if v is None:
            raise LlamaGgufError(f"missing metadata `{key}`")
        return v

    vocab = f.get_u32("llama.vocab_size")
    if vocab is None:
        toks = f.get_strings("tokenizer.ggml.tokens")
        if toks is None:
            raise LlamaGgufError("missing metadata `llama.vocab_size`")
        vocab = len(toks)
    hidden, heads = need("llama.embedding_length"), need("llama.attention.head_count")
    hd = f.get_u32("llama.attention.key_length")
    if hd is None:
        if hidden % heads:
            raise LlamaGgufError(f"hidden size {hidden} is not a multiple of {heads} heads")
        hd = hidden // heads
    kv = need("llama.attention.head_count_kv")
    if kv == 0 or heads % kv:
        raise LlamaGgufError(f"{heads} query heads do not group over {kv} kv heads")
    return LlamaConfig(vocab=vocab, hidden=hidden, heads=heads, kv_heads=kv, head_dim=hd,
                       ffn=need("llama.feed_forward_length"), layers=need("llama.block_count"),
                       theta=need_f("llama.rope.freq_base"), eps=need_f("llama.attention.layer_norm_rms_epsilon"))


def unpermute_rope(w: np.ndarray, heads: int) -> np.ndarray:
    """gguf.rs:32-56: rows [heads * hd, cols]; row 2i + k of each head goes
    back to row k * hd/2 + i."""
    rows = w.shape[0]
    hd = rows // heads
    return w.reshape(heads, hd // 2, 2, -1).transpose(0, 2, 1, 3).reshape(w.shape)


def permute_rope(w: np.ndarray, heads: int) -> np.ndarray:
    """The converter's permutation, the inverse of `unpermute_rope`."""
    rows = w.shape[0]
    hd = rows // heads
    return w.reshape(heads, 2, hd // 2, -1).transpose(0, 2, 1, 3).reshape(w.shape)


def load_llama_gguf(path_or_file):
    """(config, weights) for `LlamaStack` from a GGUF Llama: every tensor
    decoded to f32 and checked against the geometry (weights.rs:180-230);
    `output.weight` absent means tied embeddings; `rope_freqs.weight`, when
    present (Llama-3 frequency scaling), is bound as the RoPE divisors."""
    f = path_or_file if isinstance(path_or_file, GgufFile) else GgufFile.open(path_or_file)
    c = config_from_gguf(f)
    qd, kvd = c.heads * c.head_dim, c.kv_heads * c.head_dim

    def get(name, shape):
        t = f.info(name)
        if t is None:
            raise LlamaGgufError(f"missing tensor `{name}`")
        if t.shape() != tuple(shape):
            raise LlamaGgufError(f"tensor `{name}` is {t.shape()}, wanted {tuple(shape)}")
        return f.tensor_f32(name).reshape(shape)

    w = {"embed": get("token_embd.weight", (c.vocab, c.hidden)),
         "norm": get("output_norm.weight", (c.hidden,))}
    w["lm_head"] = get("output.weight", (c.vocab, c.hidden)) if f.info("output.weight") else w["embed"]
    for l in range(c.layers):
        p = f"blk.{l}"
        w[f"{l}.attn_norm"] = get(f"{p}.attn_norm.weight", (c.hidden,))
        w[f"{l}.wq"] = unpermute_rope(get(f"{p}.attn_q.weight", (qd, c.hidden)), c.heads)
        w[f"{l}.wk"] = unpermute_rope(get(f"{p}.attn_k.weight", (kvd, c.hidden)), c.kv_heads)
        w[f"{l}.wv"] = get(f"{p}.attn_v.weight", (kvd, c.hidden))
        w[f"{l}.wo"] = get(f"{p}.attn_output.weight", (c.hidden, qd))
        w[f"{l}.ffn_norm"] = get(f"{p}.ffn_norm.weight", (c.hidden,))
        w[f"{l}.wg"] = get(f"{p}.ffn_gate.weight", (c.ffn, c.hidden))
        w[f"{l}.wu"] = get(f"{p}.ffn_up.weight", (c.ffn, c.hidden))
        w[f"{l}.wd"] = get(f"{p}.ffn_down.weight", (c.hidden, c.ffn))
    if f.info("rope_freqs.weight") is not None:
        w["rope_freqs"] = get("rope_freqs.weight", (c.head_dim // 2,))
    return c, {k: np.ascontiguousarray(v, np.float32) for k, v in w.items()}
