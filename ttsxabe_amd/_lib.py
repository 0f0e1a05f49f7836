"""Loads libllmtie_hip.so and declares the C ABI of include/llmtie_hip.h.

torch is imported first on purpose: its bundled HIP runtime (SONAME
libamdhip64.so.7) is then the one the library binds to, so device pointers and
streams from torch are valid in the library's launches.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import torch  # noqa: F401  (see module docstring)

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libllmtie_hip.so"

P = C.c_void_p
SZ = C.c_size_t
I = C.c_int
F = C.c_float


class LlmtieError(C.Structure):
    _fields_ = [("status", C.c_int), ("field", SZ * 4), ("message", C.c_char * 240)]


# name -> (restype, argtypes), in header order.
SIGNATURES = {
    "llmtie_last_error": (I, [P]),
    "llmtie_version": (C.c_char_p, []),
    "llmtie_decode_scratch_new": (P, []),
    "llmtie_decode_scratch_free": (None, [P]),
    "llmtie_decode_scratch_status": (I, [P]),
    "llmtie_debug_fake_xcc": (None, [I]),
    "llmtie_supports_flash": (I, [SZ, SZ, SZ]),
    "llmtie_flash_attn": (I, [P, P, SZ, P, SZ, P, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, SZ, F, I]),
    "llmtie_flash_attn_f16": (I, [P, P, SZ, P, SZ, P, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, SZ, F, I]),
    "llmtie_flash_attn_rows": (I, [P, P, SZ, P, SZ, SZ, SZ, SZ, F]),
    "llmtie_attn_decode_f16": (I, [P, P, SZ, P, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, F, I, P, P, SZ]),
    "llmtie_attn_decode_f16_noalloc": (I, [P, P, SZ, P, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, F, I, P, SZ]),
    "llmtie_attn_decode_f16_q": (I, [P, P, SZ, P, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, F, I, P, P, SZ, P, SZ]),
    "llmtie_attn_decode_f16_q_row": (I, [P, P, SZ, SZ, P, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, F, I, P, P, SZ, P, SZ,
                                         SZ, SZ]),
    "llmtie_attn_decode": (I, [P, P, SZ, P, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, F, I, P, P, SZ]),
    "llmtie_attn_decode_q8_batch": (I, [P, P, SZ, P, SZ, SZ, P, P, SZ, SZ, SZ, SZ, SZ, SZ, F, I, P, P, SZ]),
    "llmtie_t16_cache_len": (SZ, [SZ, SZ, SZ]),
    "llmtie_t16_append": (I, [P, P, SZ, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, I]),
    "llmtie_t16_rope_cache": (I, [P, P, SZ, SZ, P, SZ, SZ, P, SZ, SZ, P, SZ, SZ, SZ, F, SZ, P, SZ, SZ]),
    "llmtie_t16_grow": (I, [P, P, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ]),
    "llmtie_t16_from_ref": (I, [P, P, SZ, P, SZ, SZ, SZ, SZ, SZ, P, SZ]),
    "llmtie_attn_decode_t16": (I, [P, P, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, F, I, P, P, SZ]),
    "llmtie_attn_decode_t16_q_row": (I, [P, P, SZ, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, F, I, P, P, SZ, P, SZ, SZ, SZ]),
    "llmtie_flash_attn_t16": (I, [P, P, SZ, P, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, SZ, F, I]),
    "llmtie_rope": (I, [P, P, SZ, SZ, P, SZ, SZ, SZ, F, SZ]),
    "llmtie_cache_append": (I, [P, P, SZ, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, I]),
    "llmtie_cache_append_f16": (I, [P, P, SZ, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, I]),
    "llmtie_rope_cache_f16": (I, [P, P, SZ, SZ, P, SZ, SZ, P, SZ, SZ, P, SZ, SZ, SZ, F, SZ, P, P, SZ, SZ]),
    "llmtie_cache_grow": (I, [P, P, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, I]),
    "llmtie_cache_grow_f16": (I, [P, P, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, I]),
    "llmtie_q8_cache_bytes": (SZ, [SZ, SZ, SZ, SZ]),
    "llmtie_kv_q8_append": (I, [P, P, SZ, SZ, P, SZ, SZ, P, SZ, SZ, SZ, SZ, SZ, SZ, SZ, SZ]),
    "llmtie_rope_cache_q8": (I, [P, P, SZ, SZ, P, SZ, SZ, P, SZ, SZ, P, SZ, SZ, SZ, F, SZ, P, SZ, SZ, SZ, SZ]),
}

_lib = None


def lib():
    """The loaded library. Raises if it has not been built: there is no
    fallback path."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m ttsxabe_amd.build` (or __graft_entry__.build())")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib
