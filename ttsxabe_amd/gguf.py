"""GGUF v3 container reading (and writing) for the weights around the path.

The reference reads its chat model's weights out of a GGUF
(crates/llmtie-gguf: `GgufFile` in src/file.rs, the block formats in
src/dequant.rs, the type table in src/types.rs); this module is the same
contract for the layer stack here: addressing and validation, the metadata
store, the tensor directory, and each tensor's bytes as f32 or f16.

Container (file.rs:430-520): "GGUF", u32 version (3 only), u64 tensor count,
u64 metadata count, that many (string key, u32 type tag, value) pairs, that
many tensor records (string name, u32 rank <= 4, u64 dims fastest-varying
first, u32 ggml type, u64 offset into the data section), then padding to
`general.alignment` (default 32, a power of two) and the data section.
Strings are a u64 length and UTF-8 bytes; arrays a u32 element tag, a u64
count and the elements (no arrays of arrays). Everything is little-endian.

Every check the reference makes at open is made here, with the same error
variants (error.rs): bad magic, other versions, truncation, bad UTF-8,
unknown value tags, nested arrays, duplicate keys and tensors, a
non-power-of-two alignment, rank > 4, unknown type ids, a fastest dimension
that is not whole blocks, and a tensor reaching past the end of the file.

Decoded to f32 exactly as the reference does: F32, F16, BF16 (exact widenings),
Q8_0 (d * q), Q4_0 (d * (q - 8)), Q4_1 (d * q + m), Q5_0 (d * (q - 16)) and
Q5_1 (d * q + m), with the 4-bit codes of a 32-block's first 16 values in the
low nibbles and of the last 16 in the high nibbles, and Q5's fifth bit j in
bit j of the little-endian u32 `qh` (dequant.rs:121-185). The K-quants
(Q2_K .. Q6_K) are sized and addressed but not decoded: this module raises
`UnsupportedGgmlType` for them at decode time (their layouts are pinned in
the reference only by a captured corpus this tree does not hold).

The file is memory-mapped (numpy.memmap): opening a large checkpoint touches
the pages the directory scan needs and nothing else.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

GGUF_VERSION = 3
DEFAULT_ALIGNMENT = 32
GGML_MAX_DIMS = 4

# ggml type id -> (name, elements per block, bytes per block)  (types.rs:19-106)
GGML_TYPES = {
    0: ("F32", 1, 4),
    1: ("F16", 1, 2),
    2: ("Q4_0", 32, 18),
    3: ("Q4_1", 32, 20),
    6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24),
    8: ("Q8_0", 32, 34),
    10: ("Q2_K", 256, 84),
    11: ("Q3_K", 256, 110),
    12: ("Q4_K", 256, 144),
    13: ("Q5_K", 256, 176),
    14: ("Q6_K", 256, 210),
    30: ("BF16", 1, 2),
}
GGML_ID = {v[0]: k for k, v in GGML_TYPES.items()}
DECODED = {"F32", "F16", "BF16", "Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0"}

# Metadata value tags (file.rs:380-402).
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", U64: "<Q", I64: "<q",
           F64: "<d"}


class GgufError(Exception):
    """Base of the reader's errors (crates/llmtie-gguf/src/error.rs)."""


class BadMagic(GgufError):
    def __init__(self, magic: bytes):
        super().__init__(f"not a GGUF file: magic is {magic!r}, wanted b'GGUF'")
        self.magic = magic


class UnsupportedVersion(GgufError):
    def __init__(self, version: int):
        super().__init__(f"GGUF version {version} is not supported; this reader is v3 only")
        self.version = version


class UnexpectedEof(GgufError):
    def __init__(self, context: str, offset: int):
        super().__init__(f"unexpected end of file reading {context} at byte {offset}")
        self.context, self.offset = context, offset


class InvalidUtf8(GgufError):
    def __init__(self):
        super().__init__("invalid UTF-8 in the metadata")


class UnknownValueType(GgufError):
    def __init__(self, tag: int):
        super().__init__(f"unknown metadata value type {tag}")
        self.tag = tag


class NestedArray(GgufError):
    def __init__(self):
        super().__init__("nested arrays are not part of GGUF")


class DuplicateKey(GgufError):
    def __init__(self, key: str):
        super().__init__(f"duplicate metadata key `{key}`")
        self.key = key


class DuplicateTensor(GgufError):
    def __init__(self, name: str):
        super().__init__(f"duplicate tensor `{name}`")
        self.name = name


class BadAlignment(GgufError):
    def __init__(self, alignment: int):
        super().__init__(f"alignment {alignment} is not a power of two")
        self.alignment = alignment


class TooManyDimensions(GgufError):
    def __init__(self, name: str, n_dims: int):
        super().__init__(f"tensor `{name}` claims {n_dims} dimensions; ggml allows at most 4")
        self.name, self.n_dims = name, n_dims


class UnsupportedGgmlType(GgufError):
    def __init__(self, name: str, ggml_type: int):
        super().__init__(f"tensor `{name}` has ggml type {ggml_type}, which this reader does not decode")
        self.name, self.ggml_type = name, ggml_type


class TensorOutOfBounds(GgufError):
    def __init__(self, name: str, start: int, end: int, file_len: int):
        super().__init__(f"tensor `{name}` spans {start}..{end} but the file is {file_len} bytes")
        self.name, self.start, self.end, self.file_len = name, start, end, file_len


class RaggedBlocks(GgufError):
    def __init__(self, name: str, row: int, block: int):
        super().__init__(f"tensor `{name}` has rows of {row}, which is not a multiple of {block}")
        self.name, self.row, self.block = name, row, block


class ShortBlockData(GgufError):
    def __init__(self, ggml_type: str, needed: int, found: int):
        super().__init__(f"{needed} bytes of {ggml_type} blocks were asked for, but only {found} were given")
        self.ggml_type, self.needed, self.found = ggml_type, needed, found


class MissingTensor(GgufError):
    def __init__(self, name: str):
        super().__init__(f"no tensor named `{name}`")
        self.name = name


@dataclass(frozen=True)
class TensorInfo:
    """One directory entry (file.rs:27-64). `dims` is ggml order (dims[0]
    varies fastest); `shape()` is the row-major reading."""
    name: str
    dims: tuple
    ggml_type: int
    offset: int
    n_elements: int
    n_bytes: int

    @property
    def type_name(self) -> str:
        return GGML_TYPES[self.ggml_type][0]

    @property
    def quantized(self) -> bool:
        return self.type_name not in ("F32", "F16", "BF16")

    def shape(self) -> tuple:
        return tuple(reversed(self.dims))


class GgufArray(list):
    """A metadata array: its items, and `etype`, the element type tag."""

    def __init__(self, etype: int, items):
        super().__init__(items)
        self.etype = etype


class _Cursor:
    def __init__(self, buf):
        self.b, self.p = buf, 0

    def take(self, n: int, context: str) -> bytes:
        if self.p + n > len(self.b):
            raise UnexpectedEof(context, self.p)
        out = bytes(self.b[self.p:self.p + n])
        self.p += n
        return out

    def scalar(self, fmt: str, context: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt), context))[0]

    def string(self, context: str) -> str:
        n = self.scalar("<Q", context)
        raw = self.take(n, context)
        try:
            return raw.decode("utf-8")
        except UnicodeDecodeError:
            raise InvalidUtf8() from None

    def value(self, tag: int, nested: bool = False):
        if tag in _SCALAR:
            return self.scalar(_SCALAR[tag], "a metadata value")
        if tag == BOOL:
            return self.take(1, "a metadata value")[0] != 0
        if tag == STRING:
            return self.string("a metadata string")
        if tag == ARRAY:
            if nested:
                raise NestedArray()
            et = self.scalar("<I", "an array type")
            n = self.scalar("<Q", "an array length")
            if et == ARRAY:
                raise NestedArray()
            if et not in _SCALAR and et not in (BOOL, STRING):
                raise UnknownValueType(et)
            return GgufArray(et, (self.value(et, True) for _ in range(n)))
        raise UnknownValueType(tag)


class GgufFile:
    """A parsed GGUF with zero-copy access to each tensor's bytes
    (file.rs:74-330). `open` maps a file; `from_bytes` parses an image."""

    def __init__(self, buf, path):
        self._buf = buf
        self.path = path
        cur = _Cursor(buf)
        magic = cur.take(4, "the magic")
        if magic != b"GGUF":
            raise BadMagic(magic)
        self.version = cur.scalar("<I", "the version")
        if self.version != GGUF_VERSION:
            raise UnsupportedVersion(self.version)
        n_tensors = cur.scalar("<Q", "the tensor count")
        n_kv = cur.scalar("<Q", "the metadata count")
        self.metadata: dict = {}
        self._tags: dict = {}
        for _ in range(n_kv):
            key = cur.string("a metadata key")
            tag = cur.scalar("<I", "a metadata type")
            val = cur.value(tag)
            if key in self.metadata:
                raise DuplicateKey(key)
            self.metadata[key] = val
            self._tags[key] = tag
        if "general.alignment" in self.metadata:
            if self._tags["general.alignment"] != U32:
                raise BadAlignment(0)
            self.alignment = self.metadata["general.alignment"]
        else:
            self.alignment = DEFAULT_ALIGNMENT
        a = self.alignment
        if a == 0 or a & (a - 1):
            raise BadAlignment(a)
        self.tensors: list = []
        self._index: dict = {}
        for _ in range(n_tensors):
            name = cur.string("a tensor name")
            n_dims = cur.scalar("<I", "a tensor rank")
            if n_dims > GGML_MAX_DIMS:
                raise TooManyDimensions(name, n_dims)
            dims = tuple(cur.scalar("<Q", "a tensor dimension") for _ in range(n_dims))
            ty = cur.scalar("<I", "a tensor type")
            if ty not in GGML_TYPES:
                raise UnsupportedGgmlType(name, ty)
            offset = cur.scalar("<Q", "a tensor offset")
            n_el = int(np.prod(dims, dtype=object)) if dims else 1
            _, bs, ts = GGML_TYPES[ty]
            if dims and dims[0] % bs:
                raise RaggedBlocks(name, dims[0], bs)
            if name in self._index:
                raise DuplicateTensor(name)
            self._index[name] = len(self.tensors)
            self.tensors.append(TensorInfo(name, dims, ty, offset, n_el, n_el // bs * ts))
        self.data_offset = -(-cur.p // a) * a
        for t in self.tensors:
            start = self.data_offset + t.offset
            end = start + t.n_bytes
            if end > len(buf):
                raise TensorOutOfBounds(t.name, start, end, len(buf))

    @classmethod
    def open(cls, path) -> "GgufFile":
        path = Path(path)
        return cls(np.memmap(path, dtype=np.uint8, mode="r"), path)

    @classmethod
    def from_bytes(cls, data: bytes) -> "GgufFile":
        return cls(np.frombuffer(data, dtype=np.uint8), Path("<memory>"))

    def __len__(self) -> int:
        return len(self.tensors)

    def info(self, name: str):
        i = self._index.get(name)
        return None if i is None else self.tensors[i]

    def keys(self):
        return self.metadata.keys()

    def get(self, key: str):
        return self.metadata.get(key)

    def get_u32(self, key: str):
        """Widens the narrower unsigned types; refuses narrowing (file.rs:216-232)."""
        v, tag = self.metadata.get(key), self._tags.get(key)
        if tag in (U8, U16, U32) or (tag in (U64, I32, I64) and 0 <= v <= 0xFFFFFFFF):
            return int(v)
        return None

    def get_f32(self, key: str):
        v, tag = self.metadata.get(key), self._tags.get(key)
        if tag in (F32, F64, U32, I32):
            return float(np.float32(v))
        return None

    def get_str(self, key: str):
        return self.metadata[key] if self._tags.get(key) == STRING else None

    def _array(self, key: str, etype: int):
        v = self.metadata.get(key)
        return list(v) if isinstance(v, GgufArray) and v.etype == etype else None

    def get_strings(self, key: str):
        return self._array(key, STRING)

    def get_f32s(self, key: str):
        return self._array(key, F32)

    def get_i32s(self, key: str):
        return self._array(key, I32)

    def tensor_bytes(self, name: str) -> np.ndarray:
        """The tensor's raw bytes, a uint8 view of the mapping."""
        t = self.info(name)
        if t is None:
            raise MissingTensor(name)
        start = self.data_offset + t.offset
        return self._buf[start:start + t.n_bytes]

    def tensor_f32(self, name: str) -> np.ndarray:
        """The tensor as f32 in file order (flat), whatever it is stored as."""
        t = self.info(name)
        if t is None:
            raise MissingTensor(name)
        return dequantize(t.type_name, self.tensor_bytes(name), t.n_elements, name)

    def tensor_f16(self, name: str) -> np.ndarray:
        """The tensor as f16 bits (uint16): F16 bytes as they are, anything
        else decoded to f32 and rounded once to nearest even (file.rs:346-390)."""
        t = self.info(name)
        if t is None:
            raise MissingTensor(name)
        raw = self.tensor_bytes(name)
        if t.type_name == "F16":
            return np.frombuffer(raw.tobytes(), dtype="<u2").copy()
        return self.tensor_f32(name).astype(np.float16).view(np.uint16)


def _f16(raw: np.ndarray, at: int) -> np.ndarray:
    """f16 at byte `at` of each block row of `raw` [blocks, type size], as f32."""
    return raw[:, at:at + 2].copy().view("<f2").astype(np.float32)


def _nibbles(qs: np.ndarray) -> np.ndarray:
    """[blocks, 16] bytes -> [blocks, 32] codes: the low nibbles are values
    0..15 of the block, the high nibbles values 16..31."""
    return np.concatenate([qs & 0x0F, qs >> 4], axis=1).astype(np.int32)


def _fifth_bits(qh: np.ndarray) -> np.ndarray:
    """[blocks, 4] bytes of a little-endian u32 -> [blocks, 32] bit j of it."""
    word = qh.copy().view("<u4").astype(np.int64)  # [blocks, 1]
    return ((word >> np.arange(32)) & 1).astype(np.int32)


def dequantize(type_name: str, raw, n: int, name: str = "<slice>") -> np.ndarray:
    """`n` values of `type_name` from `raw` bytes, as f32, the reference's
    arithmetic (dequant.rs:106-185): products and sums at f32, no fusing."""
    if type_name not in GGML_ID:
        raise GgufError(f"unknown ggml type {type_name}")
    tid = GGML_ID[type_name]
    _, bs, ts = GGML_TYPES[tid]
    if n % bs:
        raise RaggedBlocks(name, n, bs)
    need = n // bs * ts
    raw = np.asarray(raw, dtype=np.uint8).reshape(-1)
    if raw.size < need:
        raise ShortBlockData(type_name, need, int(raw.size))
    raw = raw[:need]
    if type_name == "F32":
        return raw.copy().view("<f4").astype(np.float32)
    if type_name == "F16":
        return raw.copy().view("<f2").astype(np.float32)
    if type_name == "BF16":
        return (raw.copy().view("<u2").astype(np.uint32) << 16).view(np.float32)
    if type_name not in DECODED:
        raise UnsupportedGgmlType(name, tid)
    blk = raw.reshape(-1, ts)
    f32 = np.float32
    if type_name == "Q8_0":
        d = _f16(blk, 0)
        q = blk[:, 2:].view(np.int8).astype(f32)
        out = d[:, :1] * q
    elif type_name == "Q4_0":
        d = _f16(blk, 0)
        out = d[:, :1] * (_nibbles(blk[:, 2:]) - 8).astype(f32)
    elif type_name == "Q4_1":
        d, m = _f16(blk, 0), _f16(blk, 2)
        out = (d[:, :1] * _nibbles(blk[:, 4:]).astype(f32)) + m[:, :1]
    elif type_name == "Q5_0":
        d = _f16(blk, 0)
        q = _nibbles(blk[:, 6:]) | (_fifth_bits(blk[:, 2:6]) << 4)
        out = d[:, :1] * (q - 16).astype(f32)
    else:  # Q5_1
        d, m = _f16(blk, 0), _f16(blk, 2)
        q = _nibbles(blk[:, 8:]) | (_fifth_bits(blk[:, 4:8]) << 4)
        out = (d[:, :1] * q.astype(f32)) + m[:, :1]
    return out.astype(np.float32).reshape(-1)


def write_gguf(path, metadata: dict, tensors: list, alignment: int = DEFAULT_ALIGNMENT):
    """Writes a v3 GGUF. `metadata`: key -> (tag, value); `tensors`: a list of
    (name, ggml type name, dims in ggml order, raw bytes). Tensors are laid
    out in order, each at an `alignment`-aligned offset of the data section."""
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", GGUF_VERSION, len(tensors), len(metadata))

    def put_str(s: str):
        b = s.encode("utf-8")
        out.extend(struct.pack("<Q", len(b)) + b)

    def put_val(tag: int, v):
        if tag in _SCALAR:
            out.extend(struct.pack(_SCALAR[tag], v))
        elif tag == BOOL:
            out.append(1 if v else 0)
        elif tag == STRING:
            put_str(v)
        elif tag == ARRAY:
            et, items = v
            out.extend(struct.pack("<IQ", et, len(items)))
            for x in items:
                put_val(et, x)
        else:
            raise ValueError(f"unknown tag {tag}")

    for key, (tag, v) in metadata.items():
        put_str(key)
        out.extend(struct.pack("<I", tag))
        put_val(tag, v)
    offs, off = [], 0
    for name, tname, dims, raw in tensors:
        offs.append(off)
        off = -(-(off + len(raw)) // alignment) * alignment
    for (name, tname, dims, raw), o in zip(tensors, offs):
        put_str(name)
        out.extend(struct.pack("<I", len(dims)))
        for d in dims:
            out.extend(struct.pack("<Q", d))
        out.extend(struct.pack("<IQ", GGML_ID[tname], o))
    out.extend(b"\0" * ((-len(out)) % alignment))
    base = len(out)
    for (name, tname, dims, raw), o in zip(tensors, offs):
        out.extend(b"\0" * (base + o - len(out)))
        out.extend(bytes(raw))
    Path(path).write_bytes(bytes(out))
