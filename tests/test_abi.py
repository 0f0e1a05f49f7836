"""The C ABI as a library: it loads, exports every function include/llmtie_hip.h
declares with the argument count the host binding uses, and refuses shapes
before touching a device (the reference's refusals, error.rs:148-282), so all
of this runs on a machine with no GPU."""
import ctypes as C
import re
from pathlib import Path

import pytest

from ttsxabe_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "llmtie_hip.h"


def declared():
    """name -> argument count, parsed from the header's prototypes."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|void|size_t|const char\*|llmtie_decode_scratch\*)\s+(llmtie_\w+)\s*\(([^)]*)\)\s*;",
                         text):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_header_and_binding_agree():
    d = declared()
    assert len(d) >= 30
    assert set(d) == set(_lib.SIGNATURES), set(d) ^ set(_lib.SIGNATURES)
    for name, n in d.items():
        assert len(_lib.SIGNATURES[name][1]) == n, name


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in declared():
        assert hasattr(L, name), name
    assert L.llmtie_version() == b"0.1.0"


def last():
    e = _lib.LlmtieError()
    _lib.lib().llmtie_last_error(C.byref(e))
    return e


NULL = None


def test_supports_flash_is_the_reference_predicate():
    L = _lib.lib()
    assert L.llmtie_supports_flash(128, 32, 8)
    assert L.llmtie_supports_flash(64, 20, 20)
    assert not L.llmtie_supports_flash(96, 4, 4)
    assert not L.llmtie_supports_flash(128, 4, 3)


def test_refusals_happen_before_any_launch():
    L = _lib.lib()
    # An uninstantiated head width (kernels.rs tests :2442-2473).
    assert L.llmtie_flash_attn(NULL, NULL, 10**9, NULL, 10**9, NULL, 10**9, NULL, 10**9, 4, 0, 4, 4, 96, 4,
                               C.c_float(1.0), 0) == 1
    e = last()
    assert e.status == 1 and list(e.field)[:3] == [96, 4, 4]
    assert b"head_dim 96" in e.message
    # An odd f16 capacity.
    assert L.llmtie_flash_attn_f16(NULL, NULL, 10**9, NULL, 10**9, NULL, 10**9, NULL, 10**9, 4, 0, 4, 4, 128, 7,
                                   C.c_float(1.0), 1) == 2
    # More keys than the cache holds; no keys at all (kernels.rs:2905-2937).
    for tk in (257, 0):
        assert L.llmtie_attn_decode_f16(NULL, NULL, 10**9, NULL, 10**9, NULL, 10**9, 8, 2, 128, tk, 256,
                                        C.c_float(1.0), 0, NULL, NULL, 10**9) == 3
    # A group wider than the 16 columns of the kernel's tile.
    assert L.llmtie_attn_decode_f16(NULL, NULL, 10**9, NULL, 10**9, NULL, 10**9, 34, 2, 128, 10, 256,
                                    C.c_float(1.0), 0, NULL, NULL, 10**9) == 1
    # A short cache slice.
    assert L.llmtie_attn_decode_f16(NULL, NULL, 10**9, NULL, 100, NULL, 10**9, 8, 2, 128, 10, 256,
                                    C.c_float(1.0), 0, NULL, NULL, 10**9) == 4
    assert list(last().field)[:2] == [2 * 256 * 128, 100]
    # A twin of the wrong shape (device.rs:6362-6372).
    assert L.llmtie_attn_decode_f16_q_row(NULL, NULL, 10**9, 0, NULL, 10**9, NULL, 10**9, 8, 8, 128, 37, 64,
                                          C.c_float(0.1), 0, NULL, NULL, 10**9, NULL, 1, 1024, 1) == 6
    # A rope reading past the end (kernels.rs:2212-2240), an odd rotary head.
    assert L.llmtie_rope(NULL, NULL, 32, 1, NULL, 2, 2, 8, C.c_float(1e4), 0) == 4
    assert L.llmtie_rope(NULL, NULL, 10**6, 0, NULL, 2, 2, 7, C.c_float(1e4), 0) == 7
    # Growth that shrinks or overruns.
    assert L.llmtie_cache_grow(NULL, NULL, 10**6, NULL, 10**6, 2, 4, 8, 16, 9, 0) == 3
    assert L.llmtie_cache_grow(NULL, NULL, 10**6, NULL, 10**6, 2, 4, 16, 8, 4, 0) == 3
    # Null buffers with valid shapes are refused rather than dereferenced.
    assert L.llmtie_cache_append(NULL, NULL, 100, 0, NULL, 1000, 1, 2, 8, 8, 0, 0) == 10


def test_q8_and_tiled_sizes():
    L = _lib.lib()
    # 272 bytes per position and kv head at head_dim 128, whole 32-position blocks.
    assert L.llmtie_q8_cache_bytes(1, 1, 128, 32) == 272 * 32
    assert L.llmtie_q8_cache_bytes(2, 8, 128, 33) == 2 * 8 * 2 * 272 * 32
    assert L.llmtie_t16_cache_len(8, 128, 4096) == 8 * 4096 * 128 * 2
    assert L.llmtie_t16_cache_len(20, 64, 1500) == 20 * 47 * 32 * 64 * 2


W = 2**64  # size_t wraps here


def test_extents_that_would_wrap_are_refused():
    """Offsets and counts whose sums or products pass size_t's range must be
    refused, not wrapped into a small value that passes the length check
    (a wrapped q or out offset would read or write outside the buffer)."""
    L = _lib.lib()
    BIG = 10**9
    # q offset and out row near the top of size_t.
    assert L.llmtie_attn_decode_f16_q_row(NULL, NULL, BIG, W - 512, NULL, BIG, NULL, BIG, 4, 4, 128, 10, 64,
                                          C.c_float(0.1), 0, NULL, NULL, BIG, NULL, 0, 0, 0) == 4
    assert L.llmtie_attn_decode_f16_q_row(NULL, NULL, BIG, 0, NULL, BIG, NULL, BIG, 4, 4, 128, 10, 64,
                                          C.c_float(0.1), 0, NULL, NULL, BIG, NULL, 0, 0, W // 512) == 4
    # A twin whose rows * width wraps (its scales would sit at a wrapped address).
    assert L.llmtie_attn_decode_f16_q_row(NULL, NULL, BIG, 0, NULL, BIG, NULL, BIG, 4, 4, 128, 10, 64,
                                          C.c_float(0.1), 0, NULL, NULL, BIG, NULL, W // 512 + 1, 512, 0) == 4
    # past + tq past the top of size_t; heads * head_dim past it.
    assert L.llmtie_flash_attn(NULL, NULL, BIG, NULL, BIG, NULL, BIG, NULL, BIG, 1, W - 1, 4, 4, 64, 64,
                               C.c_float(1.0), 1) == 3
    assert L.llmtie_flash_attn(NULL, NULL, BIG, NULL, BIG, NULL, BIG, NULL, BIG, 4, 0, 2**58, 2**58, 64, 64,
                               C.c_float(1.0), 1) == 4
    assert L.llmtie_flash_attn_rows(NULL, NULL, BIG, NULL, BIG, 16, 2**58, 64, C.c_float(1.0)) == 4
    # Producers: a wrapping source offset, a wrapping rope offset.
    assert L.llmtie_cache_append(NULL, NULL, BIG, W - 8, NULL, BIG, 1, 2, 8, 16, 0, 0) == 4
    assert L.llmtie_rope(NULL, NULL, BIG, W - 8, NULL, 1, 2, 8, C.c_float(1e4), 0) == 4
    assert L.llmtie_kv_q8_append(NULL, NULL, BIG, W - 8, NULL, BIG, 0, NULL, BIG, 1, 0, 1, 2, 128, 64, 0) == 4
    # Sizes that would wrap saturate.
    assert L.llmtie_q8_cache_bytes(2**40, 2**20, 128, 64) == W - 1
    assert L.llmtie_t16_cache_len(2**50, 128, 2**20) == W - 1


def test_the_no_allocation_decode_refuses_before_the_device():
    """A call beyond the fixed scratch is refused with LLMTIE_SCRATCH_LIMIT
    before any device call, so the refusal needs no GPU."""
    L = _lib.lib()
    BIG = 10**12
    P = 4096  # a placeholder address: the call is refused before anything is read or written
    assert L.llmtie_attn_decode_f16_noalloc(NULL, P, BIG, P, BIG, P, BIG, 512, 512, 128, 4096, 4096,
                                            C.c_float(0.1), 0, P, BIG) == 12
    e = last()
    assert e.field[2] > e.field[3]


def test_the_batched_q8_decode_refuses_groups_over_its_lds_budget():
    """The stream-K kernel keeps one tiled block per wave plus two query
    buffers of group * head_dim floats per wave in LDS; groups whose buffers
    would pass a workgroup's 160 KB are refused before any device call (16
    is the largest at head_dim 64 and 128), as are caches whose one (slot,
    kv head) run of blocks passes the kernel's 32-bit buffer range."""
    L = _lib.lib()
    BIG = 10**12
    P = 4096
    for hd in (64, 128):
        assert L.llmtie_attn_decode_q8_batch(NULL, P, BIG, P, BIG, 1, P, P, 1, 64, 17 * 2, 2, hd, 64,
                                             C.c_float(0.1), 0, P, P, BIG) == 1
        assert list(last().field)[:3] == [hd, 34, 2]
    # (2**31 / 8704) blocks of 32 positions at head_dim 128 is the range's limit.
    cap = (2**31 // 8704 + 1) * 32
    assert L.llmtie_attn_decode_q8_batch(NULL, P, BIG, P, BIG, 1, P, P, 1, 64, 32, 8, 128, cap,
                                         C.c_float(0.1), 0, P, P, BIG) == 3


def test_the_decode_boundary_accepts_its_documented_superset():
    """Wider than the reference's refusals, by design (the header says so):
    the f32-cache decode takes head_dim 128 as well as 64, and every decode
    takes GQA groups up to 16 (the reference: up to 4, 8 for its h64 g8
    kernel). Such shapes pass every shape check and reach the scratch check
    (a null scratch is refused as an invalid argument, status 10), where the
    reference would refuse them as UnsupportedAttention (status 1)."""
    L = _lib.lib()
    BIG = 10**12
    P = 4096
    # attn_decode (f32 cache) at head_dim 128, group 4.
    assert L.llmtie_attn_decode(NULL, P, BIG, P, BIG, P, BIG, 32, 8, 128, 100, 128, C.c_float(0.1), 0,
                                NULL, P, BIG) == 10
    # attn_decode_f16 at a group of 16.
    assert L.llmtie_attn_decode_f16(NULL, P, BIG, P, BIG, P, BIG, 32, 2, 128, 100, 128, C.c_float(0.1), 0,
                                    NULL, P, BIG) == 10
    # ... and still refused past 16, and at a head width with no kernel.
    assert L.llmtie_attn_decode_f16(NULL, P, BIG, P, BIG, P, BIG, 34, 2, 128, 100, 128, C.c_float(0.1), 0,
                                    NULL, P, BIG) == 1
    assert L.llmtie_attn_decode(NULL, P, BIG, P, BIG, P, BIG, 8, 8, 96, 100, 128, C.c_float(0.1), 0,
                                NULL, P, BIG) == 1


def test_a_scratch_with_no_lost_head_reports_ok():
    L = _lib.lib()
    assert L.llmtie_decode_scratch_status(NULL) == 0
