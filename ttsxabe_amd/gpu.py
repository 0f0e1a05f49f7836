"""Host-side mirror of the reference's attention operators, over the C ABI.

`Gpu` has the methods of `llmtie_cuda::Gpu` that the attention path uses
(crates/llmtie-cuda/src/device.rs:2849-3190, :5410-5470, :5697-6410), with the
same names, argument order and meaning; device slices are torch tensors on
the GPU (torch is only the allocator and the stream here). Outputs are
allocated by the callee exactly where the reference allocates them. Errors are
raised as the reference's `CudaError` variants (error.rs:148-282), before any
launch, from the library's own checks.

There is no CPU fallback: constructing a `Gpu` without the built library or
without a HIP device raises.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib

__all__ = [
    "CudaError", "UnsupportedAttention", "OddCacheCapacity", "CacheOverrun", "SliceOverrun", "RaggedBlock",
    "MismatchedQ8", "OddHeadDim", "Driver", "NoDevice", "InvalidArgument", "ScratchGrowthInCapture", "ScratchLimit",
    "SplitHeadLost",
    "DecodeScratch",
    "Q8", "KvCacheQ8",
    "TiledCache16", "Gpu",
]


class CudaError(RuntimeError):
    """Base of the named refusals (error.rs)."""

    status = -1

    def __init__(self, message: str, fields=()):
        super().__init__(message)
        self.fields = tuple(fields)


class UnsupportedAttention(CudaError):
    status = 1


class OddCacheCapacity(CudaError):
    status = 2


class CacheOverrun(CudaError):
    status = 3


class SliceOverrun(CudaError):
    status = 4


class RaggedBlock(CudaError):
    status = 5


class MismatchedQ8(CudaError):
    status = 6


class OddHeadDim(CudaError):
    status = 7


class Driver(CudaError):
    status = 8


class NoDevice(CudaError):
    status = 9


class InvalidArgument(CudaError):
    status = 10


class ScratchGrowthInCapture(CudaError):
    """A decode scratch would have to grow while its stream captures a graph."""
    status = 11


class ScratchLimit(CudaError):
    """The fixed scratch of attn_decode_f16_noalloc is too small for the call."""
    status = 12


class SplitHeadLost(CudaError):
    """An earlier decode through this scratch wrote NaN for a head whose split
    workgroups did not share an XCD (the XCD-local hand-off's self-check)."""
    status = 13


_BY_STATUS = {c.status: c for c in (UnsupportedAttention, OddCacheCapacity, CacheOverrun, SliceOverrun,
                                    RaggedBlock, MismatchedQ8, OddHeadDim, Driver, NoDevice, InvalidArgument,
                                    ScratchGrowthInCapture, ScratchLimit, SplitHeadLost)}


def _check(status: int):
    if status == 0:
        return
    err = _lib.LlmtieError()
    _lib.lib().llmtie_last_error(C.byref(err))
    cls = _BY_STATUS.get(status, CudaError)
    raise cls(err.message.decode(errors="replace"), [err.field[i] for i in range(4)])


def _p(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else C.c_void_p(t.data_ptr())


def _n(t):
    return 0 if t is None else t.numel()


def _need(t, dtypes, what):
    if t is None:
        return
    if not t.is_cuda:
        raise InvalidArgument(f"{what} is not a device tensor")
    if t.dtype not in dtypes:
        raise InvalidArgument(f"{what} has dtype {t.dtype}, wanted one of {dtypes}")
    if not t.is_contiguous():
        raise InvalidArgument(f"{what} is not contiguous")


_F32 = (torch.float32,)
_H16 = (torch.float16, torch.int16, torch.uint16) if hasattr(torch, "uint16") else (torch.float16, torch.int16)
_I8 = (torch.int8,)
_I32 = (torch.int32,)


class DecodeScratch:
    """What the decode keeps between calls (device.rs:208-231): split partials
    and arrival counters, caller-owned, grown on demand."""

    def __init__(self):
        self._h = _lib.lib().llmtie_decode_scratch_new()
        if not self._h:
            raise Driver("could not allocate a decode scratch")

    @property
    def handle(self):
        return self._h

    def check(self):
        """Raises SplitHeadLost if an earlier decode through this scratch lost
        a head to the XCD-local check (read after a synchronisation); the
        status is cleared."""
        _check(_lib.lib().llmtie_decode_scratch_status(self._h))

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            try:
                _lib.lib().llmtie_decode_scratch_free(h)
            except Exception:
                pass


@dataclass
class Q8:
    """An int8 twin: `rows * k` codes then `rows * k / 32` f32 scales in one
    buffer (device.rs:498-520)."""

    buf: torch.Tensor
    rows: int
    k: int

    def scale_offset(self) -> int:
        return self.rows * self.k

    def shape(self):
        return (self.rows, self.k)

    def parts(self):
        """(codes int8 [rows*k], scales f32 [rows*k/32]) on the host."""
        raw = self.buf.cpu()
        codes = raw[: self.scale_offset()].clone()
        scales = raw[self.scale_offset(): self.scale_offset() + self.rows * self.k // 32 * 4].view(torch.float32)
        return codes, scales.clone()


class KvCacheQ8:
    """A tiled GGUF Q8_0 KV cache for `slots` sequences (layout in
    llmtie_hip.h / csrc/kvlayout.h): one int8 buffer of whole 32-position
    blocks, codes and f16 scales of K and V per block."""

    def __init__(self, slots: int, kv_heads: int, head_dim: int, cap: int, device="cuda"):
        self.slots, self.kv_heads, self.head_dim, self.cap = slots, kv_heads, head_dim, cap
        n = _lib.lib().llmtie_q8_cache_bytes(slots, kv_heads, head_dim, cap)
        self.data = torch.zeros(n, dtype=torch.int8, device=device)
        # An empty cache holds code 0 (offset-binary 0x80) with scale 0.
        blocks = self.data.view(-1, n // (slots * kv_heads * ((cap + 31) // 32)))
        blocks[:, : 64 * head_dim].fill_(-128)

    def bytes_per_position(self) -> int:
        """HBM bytes one live position of one sequence costs a decode step."""
        return 2 * self.kv_heads * (self.head_dim + 2 * self.head_dim // 32)


class TiledCache16:
    """A tiled f16 KV cache for one layer: K and V of every kv head in one
    buffer, 32-position blocks in MFMA fragment order."""

    def __init__(self, kv_heads: int, head_dim: int, cap: int, device="cuda", zero=True):
        self.kv_heads, self.head_dim, self.cap = kv_heads, head_dim, cap
        n = _lib.lib().llmtie_t16_cache_len(kv_heads, head_dim, cap)
        alloc = torch.zeros if zero else torch.empty
        self.data = alloc(n, dtype=torch.float16, device=device)


class Gpu:
    """The attention operators of `llmtie_cuda::Gpu`, on gfx950."""

    def __init__(self, device: int = 0):
        L = _lib.lib()  # raises if the library is not built
        if not torch.cuda.is_available():
            raise NoDevice("no usable HIP device")
        self.device = torch.device("cuda", device)
        self._L = L

    def _stream(self):
        return C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)

    # ------------------------------------------------------------- prefill

    def supports_flash(self, head_dim: int, heads: int, kv_heads: int) -> bool:
        return bool(self._L.llmtie_supports_flash(head_dim, heads, kv_heads))

    def _flash(self, fn, q, k, v, tq, past, heads, kv_heads, head_dim, cap, scale, causal, kdt):
        _need(q, _F32, "q")
        _need(k, kdt, "k")
        _need(v, kdt, "v")
        out = torch.empty(max(tq * heads * head_dim, 1), dtype=torch.float32, device=self.device)
        _check(fn(self._stream(), _p(q), _n(q), _p(k), _n(k), _p(v), _n(v), _p(out), tq * heads * head_dim, tq, past,
                  heads, kv_heads, head_dim, cap, C.c_float(scale), int(bool(causal))))
        return out[: tq * heads * head_dim]

    def flash_attn(self, q, k, v, tq, past, heads, kv_heads, head_dim, cap, scale, causal):
        """device.rs:5702."""
        return self._flash(self._L.llmtie_flash_attn, q, k, v, tq, past, heads, kv_heads, head_dim, cap, scale,
                           causal, _F32)

    def flash_attn_f16(self, q, k, v, tq, past, heads, kv_heads, head_dim, cap, scale, causal):
        """device.rs:5754. k, v: f16 caches (float16 or 16-bit integer bits)."""
        return self._flash(self._L.llmtie_flash_attn_f16, q, k, v, tq, past, heads, kv_heads, head_dim, cap, scale,
                           causal, _H16)

    def flash_attn_rows(self, qkv, t, heads, head_dim, scale):
        """device.rs:5812. Returns the f16 context [t * heads * head_dim]."""
        _need(qkv, _F32, "qkv")
        n = t * heads * head_dim
        out = torch.empty(max(n, 1), dtype=torch.float16, device=self.device)
        _check(self._L.llmtie_flash_attn_rows(self._stream(), _p(qkv), _n(qkv), _p(out), n, t, heads, head_dim,
                                              C.c_float(scale)))
        return out[:n]

    # -------------------------------------------------------------- decode

    def attn_decode_f16(self, q, k, v, heads, kv_heads, head_dim, tk, cap, scale, scale_q, scratch):
        """device.rs:5949."""
        _need(q, _F32, "q")
        _need(k, _H16, "k")
        _need(v, _H16, "v")
        n = heads * head_dim
        out = torch.empty(n, dtype=torch.float32, device=self.device)
        _check(self._L.llmtie_attn_decode_f16(self._stream(), _p(q), _n(q), _p(k), _n(k), _p(v), _n(v), heads,
                                              kv_heads, head_dim, tk, cap, C.c_float(scale), int(bool(scale_q)),
                                              scratch.handle, _p(out), n))
        return out

    def attn_decode_f16_noalloc(self, q, k, v, heads, kv_heads, head_dim, tk, cap, scale, scale_q, out=None):
        """attn_decode_f16 without a scratch: the library's fixed per-device
        scratch (no reference counterpart; for callers that cannot allocate).
        Calls that can overlap on one device race."""
        _need(q, _F32, "q")
        _need(k, _H16, "k")
        _need(v, _H16, "v")
        _need(out, _F32, "out")
        n = heads * head_dim
        if out is None:
            out = torch.empty(n, dtype=torch.float32, device=self.device)
        _check(self._L.llmtie_attn_decode_f16_noalloc(self._stream(), _p(q), _n(q), _p(k), _n(k), _p(v), _n(v),
                                                      heads, kv_heads, head_dim, tk, cap, C.c_float(scale),
                                                      int(bool(scale_q)), _p(out), _n(out)))
        return out

    def q8_zeros(self, rows: int, k: int) -> Q8:
        """device.rs:1056."""
        if k % 32 != 0:
            raise RaggedBlock(f"a row of {k} in blocks of 32", (k, 32))
        return Q8(torch.zeros(rows * k + rows * (k // 32) * 4, dtype=torch.int8, device=self.device), rows, k)

    def attn_decode_f16_q(self, q, k, v, heads, kv_heads, head_dim, tk, cap, scale, scale_q, scratch):
        """device.rs:5973: the context and its int8 twin."""
        _need(q, _F32, "q")
        _need(k, _H16, "k")
        _need(v, _H16, "v")
        n = heads * head_dim
        out = torch.empty(n, dtype=torch.float32, device=self.device)
        twin = Q8(torch.empty(n + (n // 32) * 4, dtype=torch.int8, device=self.device), 1, n)
        _check(self._L.llmtie_attn_decode_f16_q(self._stream(), _p(q), _n(q), _p(k), _n(k), _p(v), _n(v), heads,
                                                kv_heads, head_dim, tk, cap, C.c_float(scale), int(bool(scale_q)),
                                                scratch.handle, _p(out), n, _p(twin.buf), twin.buf.numel()))
        return out, twin

    def attn_decode_f16_q_row(self, q, q_off, k, v, heads, kv_heads, head_dim, tk, cap, scale, scale_q, scratch,
                              out, twin: Q8, row):
        """device.rs:6001."""
        _need(q, _F32, "q")
        _need(k, _H16, "k")
        _need(v, _H16, "v")
        _need(out, _F32, "out")
        _check(self._L.llmtie_attn_decode_f16_q_row(self._stream(), _p(q), _n(q), q_off, _p(k), _n(k), _p(v), _n(v),
                                                    heads, kv_heads, head_dim, tk, cap, C.c_float(scale),
                                                    int(bool(scale_q)), scratch.handle, _p(out), _n(out),
                                                    _p(twin.buf), twin.rows, twin.k, row))

    def attn_decode(self, q, k, v, heads, kv_heads, head_dim, tk, cap, scale, scale_q, scratch):
        """device.rs:6132: off an f32 cache."""
        _need(q, _F32, "q")
        _need(k, _F32, "k")
        _need(v, _F32, "v")
        n = heads * head_dim
        out = torch.empty(n, dtype=torch.float32, device=self.device)
        _check(self._L.llmtie_attn_decode(self._stream(), _p(q), _n(q), _p(k), _n(k), _p(v), _n(v), heads, kv_heads,
                                          head_dim, tk, cap, C.c_float(scale), int(bool(scale_q)), scratch.handle,
                                          _p(out), n))
        return out

    def attn_decode_q8_batch(self, q, cache: KvCacheQ8, tk_dev, slot_dev, max_tk, heads, scale, scale_q, scratch,
                             out=None):
        """Batched decode of len(tk_dev) sequences over a Q8_0 cache (new)."""
        _need(q, _F32, "q")
        _need(tk_dev, _I32, "tk")
        _need(slot_dev, _I32, "slot")
        nseq = tk_dev.numel()
        n = heads * cache.head_dim
        if out is None:
            out = torch.empty(max(nseq * n, 1), dtype=torch.float32, device=self.device)
        _check(self._L.llmtie_attn_decode_q8_batch(
            self._stream(), _p(q), _n(q), _p(cache.data), _n(cache.data), cache.slots, _p(tk_dev), _p(slot_dev),
            nseq, max_tk, heads, cache.kv_heads, cache.head_dim, cache.cap, C.c_float(scale), int(bool(scale_q)),
            scratch.handle, _p(out), _n(out)))
        return out[: nseq * n]

    # ---------------------------------------------------------- tiled f16

    def attn_decode_t16(self, q, cache: TiledCache16, heads, tk, scale, scale_q, scratch, out=None):
        """attn_decode_f16 (device.rs:5949) off a tiled cache."""
        _need(q, _F32, "q")
        n = heads * cache.head_dim
        if out is None:
            out = torch.empty(n, dtype=torch.float32, device=self.device)
        _check(self._L.llmtie_attn_decode_t16(self._stream(), _p(q), _n(q), _p(cache.data), _n(cache.data), heads,
                                              cache.kv_heads, cache.head_dim, tk, cache.cap, C.c_float(scale),
                                              int(bool(scale_q)), scratch.handle, _p(out), _n(out)))
        return out

    def attn_decode_t16_q_row(self, q, q_off, cache: TiledCache16, heads, tk, scale, scale_q, scratch, out,
                              twin: Q8 = None, row=0):
        """attn_decode_f16_q_row (device.rs:6001) off a tiled cache."""
        _need(q, _F32, "q")
        _need(out, _F32, "out")
        _check(self._L.llmtie_attn_decode_t16_q_row(
            self._stream(), _p(q), _n(q), q_off, _p(cache.data), _n(cache.data), heads, cache.kv_heads,
            cache.head_dim, tk, cache.cap, C.c_float(scale), int(bool(scale_q)), scratch.handle, _p(out), _n(out),
            None if twin is None else _p(twin.buf), 0 if twin is None else twin.rows,
            0 if twin is None else twin.k, row))

    def flash_attn_t16(self, q, cache: TiledCache16, tq, past, heads, scale, causal):
        """flash_attn_f16 (device.rs:5754) off a tiled cache."""
        _need(q, _F32, "q")
        n = tq * heads * cache.head_dim
        out = torch.empty(max(n, 1), dtype=torch.float32, device=self.device)
        _check(self._L.llmtie_flash_attn_t16(self._stream(), _p(q), _n(q), _p(cache.data), _n(cache.data), _p(out),
                                             n, tq, past, heads, cache.kv_heads, cache.head_dim, cache.cap,
                                             C.c_float(scale), int(bool(causal))))
        return out[:n]

    def t16_append(self, src, src_off, cache: TiledCache16, n, past, value):
        """cache_append_f16 (device.rs:2849) into a tiled cache; value selects V."""
        _need(src, _F32, "src")
        _check(self._L.llmtie_t16_append(self._stream(), _p(src), _n(src), src_off, _p(cache.data), _n(cache.data),
                                         n, cache.kv_heads, cache.head_dim, cache.cap, past, int(bool(value))))

    def t16_rope_cache(self, q, q_off, k, k_off, v, v_off, freq_div, heads, theta, pos, cache: TiledCache16):
        """rope_cache_f16 (device.rs:2915) into a tiled cache."""
        for t, w in ((q, "q"), (k, "k"), (v, "v"), (freq_div, "freq_div")):
            _need(t, _F32, w)
        _check(self._L.llmtie_t16_rope_cache(self._stream(), _p(q), _n(q), q_off, _p(k), _n(k), k_off, _p(v), _n(v),
                                             v_off, _p(freq_div), heads, cache.kv_heads, cache.head_dim,
                                             C.c_float(theta), pos, _p(cache.data), _n(cache.data), cache.cap))

    def t16_grow(self, src: TiledCache16, dst: TiledCache16, live):
        """cache_grow_f16 (device.rs:3152) between tiled caches."""
        _check(self._L.llmtie_t16_grow(self._stream(), _p(src.data), _n(src.data), _p(dst.data), _n(dst.data),
                                       src.kv_heads, src.head_dim, src.cap, dst.cap, live))

    def t16_from_ref(self, k, v, cache: TiledCache16, live):
        """Repack reference-layout f16 caches into a tiled one."""
        _need(k, _H16, "k")
        _need(v, _H16, "v")
        _check(self._L.llmtie_t16_from_ref(self._stream(), _p(k), _n(k), _p(v), _n(v), cache.kv_heads,
                                           cache.head_dim, cache.cap, live, _p(cache.data), _n(cache.data)))

    # ----------------------------------------------------------- producers

    def rope(self, x, off, t, heads, head_dim, theta, first):
        """device.rs:5410."""
        self.rope_scaled(x, off, None, t, heads, head_dim, theta, first)

    def rope_scaled(self, x, off, freq_div, t, heads, head_dim, theta, first):
        """device.rs:5430."""
        _need(x, _F32, "x")
        _need(freq_div, _F32, "freq_div")
        _check(self._L.llmtie_rope(self._stream(), _p(x), _n(x), off, _p(freq_div), t, heads, head_dim,
                                   C.c_float(theta), first))

    def cache_append(self, src, src_off, dst, n, kv_heads, head_dim, cap, past, transposed):
        """device.rs:3013."""
        _need(src, _F32, "src")
        _need(dst, _F32, "dst")
        _check(self._L.llmtie_cache_append(self._stream(), _p(src), _n(src), src_off, _p(dst), _n(dst), n, kv_heads,
                                           head_dim, cap, past, int(bool(transposed))))

    def cache_append_f16(self, src, src_off, dst, n, kv_heads, head_dim, cap, past, transposed):
        """device.rs:2849."""
        _need(src, _F32, "src")
        _need(dst, _H16, "dst")
        _check(self._L.llmtie_cache_append_f16(self._stream(), _p(src), _n(src), src_off, _p(dst), _n(dst), n,
                                               kv_heads, head_dim, cap, past, int(bool(transposed))))

    def rope_cache_f16(self, q, q_off, k, k_off, v, v_off, freq_div, heads, kv_heads, head_dim, theta, pos, kc, vc,
                       cap):
        """device.rs:2915 (the reference passes the projections as (buffer,
        offset) pairs; here as three tensors that may be the same one)."""
        for t, w in ((q, "q"), (k, "k"), (v, "v"), (freq_div, "freq_div")):
            _need(t, _F32, w)
        _need(kc, _H16, "kc")
        _need(vc, _H16, "vc")
        _check(self._L.llmtie_rope_cache_f16(self._stream(), _p(q), _n(q), q_off, _p(k), _n(k), k_off, _p(v), _n(v),
                                             v_off, _p(freq_div), heads, kv_heads, head_dim, C.c_float(theta), pos,
                                             _p(kc), _p(vc), min(_n(kc), _n(vc)), cap))

    def cache_grow(self, src, dst, kv_heads, head_dim, cap, new_cap, live, transposed):
        """device.rs:3086."""
        _need(src, _F32, "src")
        _need(dst, _F32, "dst")
        _check(self._L.llmtie_cache_grow(self._stream(), _p(src), _n(src), _p(dst), _n(dst), kv_heads, head_dim, cap,
                                         new_cap, live, int(bool(transposed))))

    def cache_grow_f16(self, src, dst, kv_heads, head_dim, cap, new_cap, live, transposed):
        """device.rs:3152."""
        _need(src, _H16, "src")
        _need(dst, _H16, "dst")
        _check(self._L.llmtie_cache_grow_f16(self._stream(), _p(src), _n(src), _p(dst), _n(dst), kv_heads, head_dim,
                                             cap, new_cap, live, int(bool(transposed))))

    def kv_q8_append(self, k, k_off, v, v_off, cache: KvCacheQ8, slot, n, past):
        """Quantize n rows of k and v into slot `slot` at positions past.. (new)."""
        _need(k, _F32, "k")
        _need(v, _F32, "v")
        _check(self._L.llmtie_kv_q8_append(self._stream(), _p(k), _n(k), k_off, _p(v), _n(v), v_off, _p(cache.data),
                                           _n(cache.data), cache.slots, slot, n, cache.kv_heads, cache.head_dim,
                                           cache.cap, past))

    def rope_cache_q8(self, q, q_off, k, k_off, v, v_off, freq_div, heads, theta, pos, cache: KvCacheQ8, slot):
        """The Q8_0 twin of rope_cache_f16 (new)."""
        for t, w in ((q, "q"), (k, "k"), (v, "v"), (freq_div, "freq_div")):
            _need(t, _F32, w)
        _check(self._L.llmtie_rope_cache_q8(self._stream(), _p(q), _n(q), q_off, _p(k), _n(k), k_off, _p(v), _n(v),
                                            v_off, _p(freq_div), heads, cache.kv_heads, cache.head_dim,
                                            C.c_float(theta), pos, _p(cache.data), _n(cache.data), cache.slots, slot,
                                            cache.cap))
