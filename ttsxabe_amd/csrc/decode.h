// Launch interface of the decode attention kernel (decode.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmtie {

enum KvKind { KV_F16 = 0, KV_F32 = 1, KV_T16 = 2, KV_TQ8 = 3 };

// Upper bounds on splits per head: the merging workgroup keeps (m, l) per
// split and query head in LDS, at most DECODE_MAX_SPLIT_ROWS of them.
constexpr int DECODE_MAX_SPLITS = 256;
constexpr int DECODE_MAX_SPLIT_ROWS = 1024;

// Arrival counters sit a 256-byte line apart: counters sharing a line
// serialise every workgroup's atomic at one memory channel.
constexpr int CTR_STRIDE = 64;

struct DecodeArgs {
    const float* q;          // query rows, f32
    const void* k;           // K values (reference layouts) or the tiled block array
    const void* v;           // V^T values (reference layouts); unused for tiled layouts
    float* out;              // context rows, f32
    int8_t* twin_codes;      // int8 twin of the context, or null
    float* twin_scales;      // its per-32 scales
    float* part;             // split partials: O area, then the (m, l) area at ml_off
    long ml_off;             // floats from part to the (m, l) area
    long ml_stride;          // floats of the (m, l) area per (sequence, kv head): whole 256-byte lines
    unsigned* ctr;           // arrival counters, one per (sequence, kv head) every CTR_STRIDE words, zero between calls
    const int* tk_arr;       // per-sequence live lengths (batched) or null
    const int* slot_arr;     // per-sequence cache slot (batched) or null
    long q_off, q_stride;    // element offset of sequence 0's query; elements per sequence
    long out_off, out_stride;
    int tk;                  // live length, or the bound every tk_arr entry is clamped to
    int slots;               // cache slots (batched)
    int cap;                 // positions per cache row (tiled: rounded up to whole blocks)
    int kv_heads;            // kv heads per slot
    int group;               // query heads per kv head (<= 16)
    float score_l2;          // raw dot product -> log2-unit score
    float qscale;            // applied to q before it is split
    int nit;                 // 32-key blocks per wave per split
    int splits;              // grid.x: splits of the longest sequence
    int two_phase;           // merge in a second launch (else the last split's workgroup merges)
    // Stream-K batch (sk != 0, Q8_0 cache, nseq <= 64): a 1-D grid of
    // `items` workgroups whose waves each take an equal range of the batch's
    // (sequence, kv head, 32-key block) list. Partial slots: two per wave, O
    // [16][hd] floats each, then the (m, l) area at ml_off, 32 floats each.
    int sk, nseq, items;
    // XCD-local split hand-off (xcd != 0; host-planned grid, in-launch
    // merge): a 1-D grid whose workgroup L runs item (L % 8) * (grid / 8) +
    // L / 8 (sequence-major, then kv head, then split). Workgroups are dealt
    // to the XCDs round-robin and the host sets xcd only when every XCD's run
    // of items holds whole heads, so a head's splits, partials and merge all
    // stay in one XCD's L2: plain partial stores, L2 reads in the merge.
    // The dispatcher is only relied on for workgroups L and L + 8k sharing an
    // XCD (which one a launch starts on varies with what ran before). Each
    // workgroup adds its hardware XCC id to the head's arrival counter, so
    // the merging workgroup sees whether the head really stayed on one XCD;
    // if not, the head's context is written as NaN, never silently wrong.
    int xcd;
    int xcd_fake;  // tests only: report XCC id (L / 8) % 8 instead of the real one
    // Pinned host word set (system scope) when a head's check fails, or null.
    unsigned* lost;
    // Workgroups of the launch / 8, set by launch_decode: the kernel reads it
    // with its other arguments rather than from the dispatch packet (a second
    // scalar-memory round trip before the first K/V load).
    int grid8;
};

// LDS of the stream-K batched Q8_0 kernel (four waves, each with one ring
// slot of a whole tiled block and two raw query buffers of group * hd
// floats), against the 160 KB a gfx950 workgroup can hold. The kernel
// static_asserts its ring plus the largest query buffers fits; the entry
// point refuses any group whose buffers would not (sk_group_max).
constexpr size_t SK_LDS_MAX = 160 * 1024;
constexpr int SK_WAVES = 4;
constexpr size_t sk_block_bytes(int hd) { return 2 * 32 * (size_t)hd + 2 * 32 * (size_t)(hd / 32) * 2; }
constexpr size_t sk_qdyn_bytes(int hd, int group) { return (size_t)SK_WAVES * 2 * group * hd * sizeof(float); }
constexpr size_t sk_lds_bytes(int hd, int group) { return SK_WAVES * sk_block_bytes(hd) + sk_qdyn_bytes(hd, group); }
constexpr size_t sk_qdyn_max(int hd) { return sk_qdyn_bytes(hd, 16); }
// The largest GQA group whose stream-K launch fits the LDS (16 at hd 64 and 128).
constexpr int sk_group_max(int hd) {
    int g = 16;
    while (g > 0 && sk_lds_bytes(hd, g) > SK_LDS_MAX) --g;
    return g;
}
static_assert(sk_group_max(64) == 16 && sk_group_max(128) == 16, "stream-K groups up to 16 fit the LDS");

hipError_t launch_decode(int hd, int kind, const DecodeArgs& a, int kv_heads, int nseq, hipStream_t st);

// Fills n words with v (a kernel, so it may sit inside a captured graph).
hipError_t launch_fill_u32(unsigned* p, size_t n, unsigned v, hipStream_t st);

}  // namespace llmtie
