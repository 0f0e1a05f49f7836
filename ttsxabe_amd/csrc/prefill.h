// Launch interface of the prefill (flash) attention kernel (prefill.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmtie {

// Where K and V come from.
enum PfKind {
    PF_F16 = 0,   // f16 caches: K [kv][cap][hd], V [kv][hd][cap]
    PF_F32 = 1,   // the same layout at f32
    PF_ROWS = 2,  // columns of a stacked [t, 3d] f32 q/k/v product (Whisper encoder)
    PF_T16 = 3,   // the tiled f16 cache of kvlayout.h (k = the cache, v unused)
};

struct PrefillArgs {
    const float* q;   // [tq, qs] f32; head h at column h*hd
    const void* k;    // cache base, or the K column block of the stacked rows
    const void* v;    // cache base, or the V column block of the stacked rows
    void* out;        // [tq, os] f32, or f16 for PF_ROWS
    int tq, past, heads, kv_heads, cap;
    float scale;
    int causal;
    int gb;           // query heads per workgroup (1, 2 or 4)
    int qs;           // q row stride, elements
    int kvs;          // PF_ROWS: k/v row stride, elements
    int os;           // out row stride, elements
    int scale_q;      // the scale goes on q before rounding (else on the scores)
    size_t v_bytes;   // PF_F16: bytes of the V cache allocation (bounds the tile loads)
    int out_f16;      // fast path: write the context as f16 (else f32)
    // Fast path, set by launch_prefill: the launch is a 1-D grid whose
    // workgroup L runs item (L % 8) * (items / 8) + L / 8 of the
    // (head group, position block) list, group-major, so the eight XCDs
    // (workgroups are dealt to them round-robin) each take a contiguous run
    // of whole groups and read their K/V through their own L2 (C3 at 8192
    // rows: 767 -> 679 us).
    int xcd, nrb;
    int grid8;  // workgroups of the 1-D launch / 8 (read with the arguments, not from the dispatch packet)
    int cus;          // compute units of the device (set by the entry point)
    int light_tiles;  // fast f16 kernel, set by launch_prefill: blocks of at most this many tiles wait first (0: none)
};

// nqt: 16-query tiles per wave (1, 2 or 4). waves: 4, or 8 for the encoder
// rows at nqt 1 (otherwise ignored).
hipError_t launch_prefill(int hd, int kind, int nqt, const PrefillArgs& a, hipStream_t st, int waves = 4);

}  // namespace llmtie
