"""The GGUF reader and the Llama binding (ttsxabe_amd.gguf, .llama_gguf).

Mirrors the reference's container tests (crates/llmtie-gguf/tests/
container.rs: a hand-built file round trips, dims are the reverse of a
row-major shape, bad magic and old versions are named, a Q8_0 tensor is sized
by its block geometry, an unknown type id is refused by name and id, a
truncated data section is caught at open, f16 reaches f32 and back, a missing
tensor names itself) and its block-size table (tests/dequant.rs:155-185).
The block decoders are pinned by hand-built blocks whose expected values are
written out as numbers (so a swapped nibble half or a misplaced fifth bit
fails), Q8_0 also by the oracle's closed form. The rope un-permutation is
pinned by what it is for: an interleaved rotation over the permuted rows
equals the halves rotation (the oracle's, rope.rs:83-126) over the original
ones. The reference's corpus of captured blocks (.golden/gguf/quants) is not
in its tree, so the K-quants are not decoded here (refused by name).
"""
import struct

import numpy as np
import pytest

import oracle
from ttsxabe_amd import gguf
from ttsxabe_amd.llama_gguf import LlamaGgufError, config_from_gguf, load_llama_gguf, permute_rope, unpermute_rope


def image(dims, ty, raw, meta=b"", n_kv=0, name="t", version=3, magic=b"GGUF"):
    """A one-tensor v3 image (container.rs:32-71), `meta` pre-encoded."""
    b = bytearray(magic) + struct.pack("<IQQ", version, 1, n_kv) + meta
    b += struct.pack("<Q", len(name)) + name.encode() + struct.pack("<I", len(dims))
    for d in dims:
        b += struct.pack("<Q", d)
    b += struct.pack("<IQ", ty, 0)
    while len(b) % 32:
        b.append(0)
    return bytes(b + raw)


def kv_u32(key, v):
    return struct.pack("<Q", len(key)) + key.encode() + struct.pack("<II", 4, v)


def test_a_hand_built_file_round_trips():
    data = np.arange(6, dtype="<f4")
    f = gguf.GgufFile.from_bytes(image([2, 3], 0, data.tobytes(), kv_u32("answer", 42), 1))
    assert f.version == 3 and f.alignment == 32 and len(f) == 1
    assert f.get("answer") == 42 and f.get_u32("answer") == 42
    t = f.info("t")
    assert t.dims == (2, 3) and t.n_elements == 6 and t.n_bytes == 24 and t.type_name == "F32"
    assert np.array_equal(f.tensor_f32("t"), data)


def test_ggml_dims_are_the_reverse_of_a_row_major_shape():
    f = gguf.GgufFile.from_bytes(image([4, 7], 0, bytes(4 * 28)))
    assert f.info("t").dims == (4, 7) and f.info("t").shape() == (7, 4)


def test_bad_magic_and_old_versions_are_named():
    with pytest.raises(gguf.BadMagic) as e:
        gguf.GgufFile.from_bytes(image([1], 0, bytes(4), magic=b"XGUF"))
    assert e.value.magic == b"XGUF"
    with pytest.raises(gguf.UnsupportedVersion) as e:
        gguf.GgufFile.from_bytes(image([1], 0, bytes(4), version=2))
    assert e.value.version == 2


def test_a_quantized_tensor_is_sized_by_its_block_geometry():
    f = gguf.GgufFile.from_bytes(image([32], 8, bytes(34)))
    t = f.info("t")
    assert t.type_name == "Q8_0" and t.n_elements == 32 and t.n_bytes == 34 and t.quantized


def test_block_sizes_and_type_sizes_are_the_reference_ones():
    want = {"F32": (1, 4), "F16": (1, 2), "BF16": (1, 2), "Q4_0": (32, 18), "Q4_1": (32, 20), "Q5_0": (32, 22),
            "Q5_1": (32, 24), "Q8_0": (32, 34), "Q2_K": (256, 84), "Q3_K": (256, 110), "Q4_K": (256, 144),
            "Q5_K": (256, 176), "Q6_K": (256, 210)}
    ids = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q2_K": 10, "Q3_K": 11,
           "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "BF16": 30}
    for name, (bs, ts) in want.items():
        assert gguf.GGML_TYPES[ids[name]] == (name, bs, ts)


def test_refusals_name_what_is_wrong():
    with pytest.raises(gguf.UnsupportedGgmlType) as e:
        gguf.GgufFile.from_bytes(image([32], 16, bytes(64)))
    assert (e.value.name, e.value.ggml_type) == ("t", 16)
    with pytest.raises(gguf.TensorOutOfBounds) as e:
        gguf.GgufFile.from_bytes(image([8], 0, bytes(16)))
    assert e.value.name == "t"
    with pytest.raises(gguf.RaggedBlocks) as e:
        gguf.GgufFile.from_bytes(image([20], 8, bytes(34)))
    assert (e.value.row, e.value.block) == (20, 32)
    with pytest.raises(gguf.TooManyDimensions):
        gguf.GgufFile.from_bytes(image([1, 1, 1, 1, 1], 0, bytes(4)))
    with pytest.raises(gguf.UnexpectedEof):
        gguf.GgufFile.from_bytes(image([1], 0, bytes(4))[:30])
    two = kv_u32("k", 1) + kv_u32("k", 2)
    with pytest.raises(gguf.DuplicateKey):
        gguf.GgufFile.from_bytes(image([1], 0, bytes(4), two, 2))
    with pytest.raises(gguf.BadAlignment):
        gguf.GgufFile.from_bytes(image([1], 0, bytes(4), kv_u32("general.alignment", 24), 1))
    nested = struct.pack("<Q", 1) + b"a" + struct.pack("<IIQ", 9, 9, 0)
    with pytest.raises(gguf.NestedArray):
        gguf.GgufFile.from_bytes(image([1], 0, bytes(4), nested, 1))
    bad = struct.pack("<Q", 1) + b"a" + struct.pack("<I", 13)
    with pytest.raises(gguf.UnknownValueType):
        gguf.GgufFile.from_bytes(image([1], 0, bytes(4), bad, 1))
    utf = struct.pack("<Q", 2) + b"\xff\xfe" + struct.pack("<II", 4, 0)
    with pytest.raises(gguf.InvalidUtf8):
        gguf.GgufFile.from_bytes(image([1], 0, bytes(4), utf, 1))
    f = gguf.GgufFile.from_bytes(image([1], 0, bytes(4)))
    with pytest.raises(gguf.MissingTensor) as e:
        f.tensor_f32("nope")
    assert e.value.name == "nope"
    kq = gguf.GgufFile.from_bytes(image([256], 12, bytes(144)))
    with pytest.raises(gguf.UnsupportedGgmlType):
        kq.tensor_f32("t")


def test_duplicate_tensors_and_metadata_accessors(tmp_path):
    p = tmp_path / "m.gguf"
    meta = {"n8": (gguf.U8, 7), "n64": (gguf.U64, 1 << 40), "neg": (gguf.I32, -1), "x": (gguf.F64, 0.25),
            "s": (gguf.STRING, "llama"), "toks": (gguf.ARRAY, (gguf.STRING, ["a", "b", "c"])),
            "fs": (gguf.ARRAY, (gguf.F32, [0.5, 1.5])), "general.alignment": (gguf.U32, 64)}
    gguf.write_gguf(p, meta, [("a", "F32", (3,), np.ones(3, "<f4").tobytes()),
                              ("b", "F32", (2,), np.full(2, 2.0, "<f4").tobytes())], alignment=64)
    f = gguf.GgufFile.open(p)
    assert f.alignment == 64 and f.data_offset % 64 == 0 and f.info("b").offset == 64
    assert f.get_u32("n8") == 7 and f.get_u32("n64") is None and f.get_u32("neg") is None
    assert f.get_f32("x") == 0.25 and f.get_str("s") == "llama" and f.get_str("n8") is None
    assert f.get_strings("toks") == ["a", "b", "c"] and f.get_strings("fs") is None
    assert f.get_f32s("fs") == [0.5, 1.5]
    assert np.array_equal(f.tensor_f32("b"), [2.0, 2.0])
    raw = bytearray(p.read_bytes())
    i = raw.rindex(b"\x01\x00\x00\x00\x00\x00\x00\x00b")  # the second tensor's name "b" -> "a"
    raw[i + 8] = ord("a")
    with pytest.raises(gguf.DuplicateTensor):
        gguf.GgufFile.from_bytes(bytes(raw))


def test_f16_reaches_f32_and_back_without_a_conversion_in_the_middle():
    halves = np.array([0x3C00, 0xC100, 0x3000], np.uint16)  # 1.0, -2.5, 0.125
    f = gguf.GgufFile.from_bytes(image([3], 1, halves.astype("<u2").tobytes()))
    assert np.array_equal(f.tensor_f16("t"), halves)
    assert np.array_equal(f.tensor_f32("t"), [1.0, -2.5, 0.125])
    bf = np.array([0x3F80, 0xC020], np.uint16)  # bf16 1.0, -2.5
    g = gguf.GgufFile.from_bytes(image([2], 30, bf.astype("<u2").tobytes()))
    assert np.array_equal(g.tensor_f32("t"), [1.0, -2.5])


def test_legacy_blocks_decode_to_hand_computed_values():
    d = struct.pack("<e", 0.5)
    m = struct.pack("<e", -1.0)
    qs = bytes([0x1F] + [0x80] * 14 + [0x3C])  # byte 0: low 15, high 1; byte 15: low 12, high 3
    # Q4_0: x[j] = 0.5 * (nibble - 8); low nibbles are values 0..15, high ones 16..31.
    x = gguf.dequantize("Q4_0", np.frombuffer(d + qs, np.uint8), 32)
    assert (x[0], x[15], x[16], x[31], x[1], x[17]) == (3.5, 2.0, -3.5, -2.5, -4.0, 0.0)
    # Q4_1: x[j] = 0.5 * nibble - 1.
    x = gguf.dequantize("Q4_1", np.frombuffer(d + m + qs, np.uint8), 32)
    assert (x[0], x[15], x[16], x[31], x[1], x[17]) == (6.5, 5.0, -0.5, 0.5, -1.0, 3.0)
    # Q5_0: fifth bit j of the little-endian qh word goes to value j.
    qh = struct.pack("<I", (1 << 0) | (1 << 17) | (1 << 31))
    x = gguf.dequantize("Q5_0", np.frombuffer(d + qh + qs, np.uint8), 32)
    # value 0: 15 | 16 = 31 -> 0.5 * 15; value 17: 8 | 16 = 24 -> 4; value 31: 3 | 16 = 19 -> 1.5
    assert (x[0], x[1], x[16], x[17], x[31]) == (7.5, -8.0, -7.5, 4.0, 1.5)
    x = gguf.dequantize("Q5_1", np.frombuffer(d + m + qh + qs, np.uint8), 32)
    assert (x[0], x[1], x[16], x[17], x[31]) == (14.5, -1.0, -0.5, 11.0, 8.5)
    with pytest.raises(gguf.ShortBlockData):
        gguf.dequantize("Q8_0", np.zeros(33, np.uint8), 32)


def test_q8_0_is_the_closed_form():
    rng = np.random.default_rng(5)
    codes = rng.integers(-127, 128, 96).astype(np.int8)
    scales = oracle.f32_to_f16(np.abs(rng.standard_normal(3)).astype(np.float32) * np.float32(0.02))
    raw = b"".join(scales[i:i + 1].astype("<u2").tobytes() + codes[32 * i:32 * i + 32].tobytes() for i in range(3))
    f = gguf.GgufFile.from_bytes(image([96], 8, raw))
    assert np.array_equal(f.tensor_f32("t"), oracle.q8_0_dequant(codes, scales))


def _interleaved(x, hd, theta, pos):
    """RoPE pairing (2i, 2i+1) over rows of width hd, f64 (the rotation
    llama.cpp's GGUF weights are permuted for)."""
    y = np.array(x, np.float64).reshape(-1, hd).copy()
    inv = theta ** (-np.arange(0, hd, 2) / hd)
    c, s = np.cos(pos * inv), np.sin(pos * inv)
    a, b = y[:, 0::2].copy(), y[:, 1::2].copy()
    y[:, 0::2], y[:, 1::2] = a * c - b * s, a * s + b * c
    return y.ravel()


def _halves(x, hd, theta, pos):
    y = np.array(x, np.float64).reshape(-1, hd).copy()
    inv = theta ** (-np.arange(0, hd, 2) / hd)
    c, s = np.cos(pos * inv), np.sin(pos * inv)
    a, b = y[:, :hd // 2].copy(), y[:, hd // 2:].copy()
    y[:, :hd // 2], y[:, hd // 2:] = a * c - b * s, a * s + b * c
    return y.ravel()


def test_the_rope_permutation_turns_an_interleaved_rotation_into_the_halves_one():
    rng = np.random.default_rng(3)
    heads, hd, cols = 3, 16, 10
    w = rng.standard_normal((heads * hd, cols))
    x = rng.standard_normal(cols)
    assert np.array_equal(unpermute_rope(permute_rope(w, heads), heads), w)
    # The halves rotation is the oracle's (position 5, theta 10000): pinned
    # against it here, then the interleaved rotation over the permuted rows,
    # un-permuted, must give the same rows.
    want = _halves(w @ x, hd, 10000.0, 5)
    assert np.allclose(want, oracle.rope((w @ x).astype(np.float32), 1, heads, hd, 10000.0, 5), atol=1e-5)
    got = unpermute_rope(_interleaved(permute_rope(w, heads) @ x, hd, 10000.0, 5)[:, None], heads)[:, 0]
    assert np.allclose(got, want, atol=1e-12)


def llama_gguf(path, cfg, w, types=("F16", "Q8_0"), rope_freqs=None):
    """Writes weights `w` (the stack's naming) as a llama.cpp-style GGUF: ggml
    names, dims reversed, q/k rows permuted, norms F32, matrices alternating
    through `types`. Returns the weights as the file holds them (rounded)."""
    def enc(x, t):
        x = np.ascontiguousarray(x, np.float32)
        if t == "F32":
            return x.astype("<f4").tobytes(), x
        if t == "F16":
            h = oracle.f32_to_f16(x)
            return h.astype("<u2").tobytes(), oracle.f16_to_f32(h)
        codes, sc = oracle.q8_0_quantize(x.ravel())
        raw = b"".join(sc[i:i + 1].astype("<u2").tobytes() + codes[32 * i:32 * i + 32].tobytes()
                       for i in range(sc.size))
        return raw, oracle.q8_0_dequant(codes, sc).reshape(x.shape)

    tensors, held, k = [], {}, 0

    def put(name, key, x, t=None, heads=None):
        nonlocal k
        if t is None:
            t = types[k % len(types)]
            k += 1
        y = permute_rope(x, heads) if heads else x
        raw, back = enc(y, t)
        tensors.append((name, t, tuple(reversed(x.shape)), raw))
        held[key] = unpermute_rope(back, heads) if heads else back

    put("token_embd.weight", "embed", w["embed"])
    put("output_norm.weight", "norm", w["norm"], "F32")
    put("output.weight", "lm_head", w["lm_head"])
    for l in range(cfg.layers):
        p = f"blk.{l}"
        put(f"{p}.attn_norm.weight", f"{l}.attn_norm", w[f"{l}.attn_norm"], "F32")
        put(f"{p}.attn_q.weight", f"{l}.wq", w[f"{l}.wq"], heads=cfg.heads)
        put(f"{p}.attn_k.weight", f"{l}.wk", w[f"{l}.wk"], heads=cfg.kv_heads)
        put(f"{p}.attn_v.weight", f"{l}.wv", w[f"{l}.wv"])
        put(f"{p}.attn_output.weight", f"{l}.wo", w[f"{l}.wo"])
        put(f"{p}.ffn_norm.weight", f"{l}.ffn_norm", w[f"{l}.ffn_norm"], "F32")
        put(f"{p}.ffn_gate.weight", f"{l}.wg", w[f"{l}.wg"])
        put(f"{p}.ffn_up.weight", f"{l}.wu", w[f"{l}.wu"])
        put(f"{p}.ffn_down.weight", f"{l}.wd", w[f"{l}.wd"])
    if rope_freqs is not None:
        put("rope_freqs.weight", "rope_freqs", rope_freqs, "F32")
    meta = {"general.architecture": (gguf.STRING, "llama"),
            "llama.vocab_size": (gguf.U32, cfg.vocab), "llama.embedding_length": (gguf.U32, cfg.hidden),
            "llama.feed_forward_length": (gguf.U32, cfg.ffn), "llama.block_count": (gguf.U32, cfg.layers),
            "llama.attention.head_count": (gguf.U32, cfg.heads),
            "llama.attention.head_count_kv": (gguf.U32, cfg.kv_heads),
            "llama.attention.key_length": (gguf.U32, cfg.head_dim),
            "llama.rope.freq_base": (gguf.F32, cfg.theta),
            "llama.attention.layer_norm_rms_epsilon": (gguf.F32, cfg.eps)}
    gguf.write_gguf(path, meta, tensors)
    return held


def test_a_llama_gguf_binds_to_the_stack_weights(tmp_path):
    from oracle.stack import StackConfig, random_weights
    cfg = StackConfig(vocab=64, hidden=128, heads=4, kv_heads=2, head_dim=32, ffn=256, layers=2)
    w = random_weights(cfg, 11)
    held = llama_gguf(tmp_path / "m.gguf", cfg, w, rope_freqs=np.linspace(1, 4, 16).astype(np.float32))
    c, got = load_llama_gguf(tmp_path / "m.gguf")
    assert (c.vocab, c.hidden, c.heads, c.kv_heads, c.head_dim, c.ffn, c.layers) == \
        (cfg.vocab, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.ffn, cfg.layers)
    assert c.theta == np.float32(cfg.theta) and c.eps == np.float32(cfg.eps)
    assert set(got) == set(held)
    for k in held:
        assert np.array_equal(got[k], held[k]), k
    # Q/K went through the permutation and back: close to the originals.
    assert np.abs(got["0.wq"] - w["0.wq"]).max() < 2e-2


def test_a_gguf_that_is_not_this_llama_is_refused(tmp_path):
    p = tmp_path / "x.gguf"
    gguf.write_gguf(p, {"general.architecture": (gguf.STRING, "bert")}, [])
    with pytest.raises(LlamaGgufError, match="bert"):
        config_from_gguf(gguf.GgufFile.open(p))
    from oracle.stack import StackConfig, random_weights
    cfg = StackConfig(vocab=64, hidden=128, heads=4, kv_heads=2, head_dim=32, ffn=256, layers=1)
    w = random_weights(cfg, 12)
    w["0.wd"] = w["0.wd"][:, :128]  # ffn_down of the wrong width
    llama_gguf(tmp_path / "m.gguf", cfg, w)
    with pytest.raises(LlamaGgufError, match="ffn_down"):
        load_llama_gguf(tmp_path / "m.gguf")
