// Flash-style prefill attention for gfx950 (causal GQA, non-causal encoder).
//
// Replaces the reference's `flash_attn_impl` and its entries `flash_attn`,
// `flash_attn_h`, `flash_attn_64`, `flash_attn_64_rows`
// (crates/llmtie-cuda/src/kernels.rs:3026-3311).
//
// Arithmetic (the reference's, kernels.rs:2955-2961): q (times the scale when
// `scale_q`) rounded to f16, K and V rounded to f16, S = Q K^T accumulated at
// f32 on MFMA, the running max in log2 units with scale * log2(e) folded in,
// probabilities rounded to f16 on their way into P V, the normaliser summed at
// f32 from the unrounded probabilities, and O / l at the end.
//
// Work decomposition. A workgroup is four waves. Like the reference, the
// waves of a workgroup are the `gb` query heads of one GQA group (so one K/V
// tile in LDS serves all of them) times 4/gb position blocks. A wave owns
// 16 * NQT query positions of one head; Q lives in registers as MFMA B
// operands for the whole kernel.
//
// Per 64-key tile (staged global -> registers -> LDS, the next tile's loads in
// flight while this one is computed) a wave computes S^T = K Q^T with
// v_mfma_f32_16x16x32_f16: A = 16 keys x 32 dims read from LDS, B = 32 dims x
// 16 queries from registers, each A fragment reused across the NQT query
// tiles. A-row m of tile (half, T) is key 32*half + 8*(m/4) + 4T + m%4, which
// leaves lane l holding the scores of keys 32*half + 8*grp + 0..7 for its
// query: the B-operand slots of O^T = V^T P^T over that half's 32 keys. P is
// therefore rounded to f16 in registers and never written to LDS; the V^T
// A-operand is one 16-byte row segment of the [d][key] tile.
//
// LDS rows are XOR-swizzled by 16-byte chunk so that the eight rows one
// ds_read_b128 phase touches land on distinct banks.
#include <stdlib.h>
#include <algorithm>
#include <type_traits>
#include "common.h"
#include "prefill.h"
#include "kvlayout.h"
#include "lineorder.h"

// LDS fragment reads kept in flight ahead of the MFMAs that use them in the
// tile loop's software pipeline, at most the pipeline's reads (measured on
// MI355X: 4 -> 6 -> 10 took C3@512 14.5 -> 14.0 -> 13.8 us and C3@8192
// 631 -> 613 -> 611 us; 12 and 16 were slower again).
// Staged (f32) encoder rows: tiles whose loads are in flight ahead of the
// one being written to LDS.
#ifndef LLMTIE_PF_SPD
#define LLMTIE_PF_SPD 2
#endif
#ifndef LLMTIE_PF_SLEEP
#define LLMTIE_PF_SLEEP 27  // s_sleep units (64 clocks)
#endif
#ifndef LLMTIE_PF_PD
#define LLMTIE_PF_PD 10
#endif

namespace llmtie {

constexpr int PW = 4;    // waves per workgroup
constexpr int PT = PW * LLMTIE_WAVE;
constexpr int KT = 64;   // keys per LDS tile

// Physical 16-byte chunk of logical chunk c in K-tile row r.
template <int HD>
__device__ __forceinline__ int swz_k(int r, int c) {
    int x = (r & 3) | (((r >> 3) & 1) << 2);
    if constexpr (HD / 8 >= 16) x |= ((r >> 4) & 1) << 3;
    return c ^ x;
}
// Physical chunk of logical chunk c (8 keys) in V^T-tile row d.
__device__ __forceinline__ int swz_v(int d, int c) { return c ^ (d & 7); }

template <int HD, int KIND>
struct Stage {
    // Per thread: K chunks and V chunks of one tile, already f16.
    static constexpr int KC = KT * (HD / 8) / PT;  // K chunks per thread
    static constexpr int VC = HD * (KT / 8) / PT;  // V chunks per thread
    half8 k[KC];
    half8 v[VC];
};

template <int HD, int KIND>
__device__ __forceinline__ half8 fetch8(const void* base, size_t off, int n, bool al) {
    // Eight consecutive elements at `off`, zero past `n` valid ones.
    half8 r = zero_h8();
    if (n <= 0) return r;
    if constexpr (KIND == PF_F16) {
        const uint16_t* p = reinterpret_cast<const uint16_t*>(base) + off;
        if (n >= 8 && al) return ld_h8(p);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (j < n) r[j] = __builtin_bit_cast(half_t, p[j]);
        return r;
    } else {
        const float* p = reinterpret_cast<const float*>(base) + off;
        if (n >= 8 && al) {
            const float4 a = reinterpret_cast<const float4*>(p)[0];
            const float4 b = reinterpret_cast<const float4*>(p)[1];
            r[0] = to_h(a.x); r[1] = to_h(a.y); r[2] = to_h(a.z); r[3] = to_h(a.w);
            r[4] = to_h(b.x); r[5] = to_h(b.y); r[6] = to_h(b.z); r[7] = to_h(b.w);
            return r;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (j < n) r[j] = to_h(p[j]);
        return r;
    }
}

template <int HD, int KIND, int NQT>
__global__ __launch_bounds__(PT) void flash_prefill_kernel(PrefillArgs a) {
    constexpr int NS = HD / 32;   // contraction steps of S
    constexpr int NT = HD / 16;   // d tiles of O^T
    constexpr int QPW = 16 * NQT;
    constexpr int KCH = HD / 8;   // 16-byte chunks per K row
    using St = Stage<HD, KIND>;

    __shared__ __attribute__((aligned(16))) half_t ks[KT * HD];
    __shared__ __attribute__((aligned(16))) half_t vs[HD * KT];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int gb = a.gb;
    const int pb = QPW * (PW / gb);
    const int group = a.heads / a.kv_heads;
    // Heaviest (latest) position blocks first under a causal mask.
    const int bx = a.causal ? (int)gridDim.x - 1 - (int)blockIdx.x : (int)blockIdx.x;
    const int h = blockIdx.y * gb + wave % gb;
    const int kh = (blockIdx.y * gb) / group;
    const int bp0 = bx * pb;
    const int p0 = bp0 + (wave / gb) * QPW;
    const int ktot = a.past + a.tq;
    const int kend = a.causal ? min(ktot, a.past + bp0 + pb) : ktot;
    const int wlim = a.causal ? min(a.past + p0 + QPW - 1, ktot - 1) : ktot - 1;

    // Source addressing. Off a cache, K row p of head kh is at (kh*cap + p)*HD
    // and V^T row d at (kh*HD + d)*cap. Off rows, both are p*kvs + kh*HD.
    const bool rows = KIND == PF_ROWS;
    const size_t kbase = rows ? (size_t)kh * HD : (size_t)kh * a.cap * HD;
    const size_t vbase = rows ? (size_t)kh * HD : (size_t)kh * HD * a.cap;
    const size_t krs = rows ? (size_t)a.kvs : (size_t)HD;
    const bool kal = rows ? (a.kvs % 4 == 0) : true;
    const bool val = rows ? kal : (KIND == PF_F16 ? a.cap % 8 == 0 : a.cap % 4 == 0);
    constexpr int SK = KIND == PF_ROWS ? PF_F32 : (KIND == PF_T16 ? PF_F16 : KIND);

    // Tiled cache: a 64-key tile is two blocks; each block's K and V areas are
    // copied verbatim (16-byte chunk i of an area to LDS chunk i), so the
    // fragment reads below are lane-contiguous and conflict-free. The loads
    // are unconditional, from the block clamped to the last one holding a key
    // below kend, so they pipeline without branches; keys past the live ones
    // are handled after the data has arrived (store_tile): their scores are
    // masked to -inf, and their V chunks are zeroed there, since a tiled
    // cache may hold non-finite garbage past ktot and 0 * NaN is NaN.
    const size_t tblk = (size_t)kh * tiled_nblk(a.cap);  // first block of this kv head
    const int lastb = (max(kend, 1) - 1) >> 5;            // last block with a key below kend
    auto load_tile = [&](int kv0, St& st) {
        if constexpr (KIND == PF_T16) {
            constexpr int AREA = 32 * HD / 8;  // 16-byte chunks per area
            static_assert(PT % AREA == 0 || AREA % PT == 0, "a chunk's block index must be wave-uniform");
            const half8* base = reinterpret_cast<const half8*>(a.k) + tblk * (2 * AREA);
#pragma unroll
            for (int i = 0; i < St::KC; ++i) {
                const int id = tid + PT * i;       // 0 .. 2*AREA-1 over the two blocks
                const int hb = id / AREA, ci = id % AREA;
                const int b = min((kv0 >> 5) + hb, lastb);
                st.k[i] = base[(size_t)b * (2 * AREA) + ci];
            }
#pragma unroll
            for (int i = 0; i < St::VC; ++i) {
                const int id = tid + PT * i;
                const int hb = id / AREA, ci = id % AREA;
                const int b = min((kv0 >> 5) + hb, lastb);
                st.v[i] = base[(size_t)b * (2 * AREA) + AREA + ci];
            }
        } else {
#pragma unroll
            for (int i = 0; i < St::KC; ++i) {
                const int id = tid + PT * i;
                const int r = id / KCH, c = id % KCH;
                st.k[i] = fetch8<HD, SK>(a.k, kbase + (size_t)(kv0 + r) * krs + 8 * c, kv0 + r < kend ? 8 : 0, kal);
            }
#pragma unroll
            for (int i = 0; i < St::VC; ++i) {
                const int id = tid + PT * i;
                if constexpr (KIND == PF_ROWS) {
                    // V rows [key][d]: chunk = 8 dims of one key.
                    const int r = id / KCH, c = id % KCH;
                    st.v[i] = fetch8<HD, SK>(a.v, vbase + (size_t)(kv0 + r) * krs + 8 * c, kv0 + r < kend ? 8 : 0, val);
                } else {
                    const int d = id / (KT / 8), c = id % (KT / 8);
                    const int p = kv0 + 8 * c;
                    st.v[i] = fetch8<HD, SK>(a.v, vbase + (size_t)d * a.cap + p, min(8, kend - p), val);
                }
            }
        }
    };
    auto store_tile = [&](int kv0, const St& st) {
        if constexpr (KIND == PF_T16) {
            constexpr int AREA = 32 * HD / 8;
#pragma unroll
            for (int i = 0; i < St::KC; ++i) {
                const int id = tid + PT * i;
                reinterpret_cast<half8*>(ks)[id] = st.k[i];  // block hb's K area at [hb * AREA]
            }
#pragma unroll
            for (int i = 0; i < St::VC; ++i) {
                const int id = tid + PT * i;
                half8 x = st.v[i];
                const int b0 = kv0 + 32 * (id / AREA);  // uniform: AREA is a multiple of the wave
                if (b0 + 32 > ktot) {                   // the tail block, or one wholly past ktot
                    const int k0 = b0 + 8 * (((id % AREA) & 63) >> 4);  // keys k0 .. k0 + 7
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        if (k0 + j >= ktot) x[j] = (half_t)0.0f;
                }
                reinterpret_cast<half8*>(vs)[id] = x;
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < St::KC; ++i) {
            const int id = tid + PT * i;
            const int r = id / KCH, c = id % KCH;
            *reinterpret_cast<half8*>(&ks[r * HD + 8 * swz_k<HD>(r, c)]) = st.k[i];
        }
#pragma unroll
        for (int i = 0; i < St::VC; ++i) {
            const int id = tid + PT * i;
            if constexpr (KIND == PF_ROWS) {
                const int key = id / KCH, c = id % KCH;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int d = 8 * c + j;
                    vs[d * KT + 8 * swz_v(d, key >> 3) + (key & 7)] = st.v[i][j];
                }
            } else {
                const int d = id / (KT / 8), c = id % (KT / 8);
                *reinterpret_cast<half8*>(&vs[d * KT + 8 * swz_v(d, c)]) = st.v[i];
            }
        }
    };
    // Fragment reads: A operand of S^T for (half, T, step) and of O^T for (half, tile).
    auto kfrag = [&](int hf, int T, int s) -> half8 {
        if constexpr (KIND == PF_T16) {
            return reinterpret_cast<const half8*>(ks)[hf * (32 * HD / 8) + (T * NS + s) * 64 + lane];
        } else {
            const int r = 32 * hf + 8 * (col >> 2) + 4 * T + (col & 3);
            return *reinterpret_cast<const half8*>(&ks[r * HD + 8 * swz_k<HD>(r, 4 * s + grp)]);
        }
    };
    auto vfrag = [&](int hf, int t) -> half8 {
        if constexpr (KIND == PF_T16) {
            return reinterpret_cast<const half8*>(vs)[hf * (32 * HD / 8) + t * 64 + lane];
        } else {
            const int d = 16 * t + col;
            return *reinterpret_cast<const half8*>(&vs[d * KT + 8 * swz_v(d, 4 * hf + grp)]);
        }
    };

    // Q as B operands: qb[u][s] holds dims 32s + 8grp + 0..7 of query p0 + 16u + col.
    const float qsc = a.scale_q ? a.scale : 1.0f;
    half8 qb[NQT][NS];
#pragma unroll
    for (int u = 0; u < NQT; ++u) {
        const int r = p0 + 16 * u + col;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            half8 x = zero_h8();
            if (r < a.tq) {
                const float4* p = reinterpret_cast<const float4*>(a.q + (size_t)r * a.qs + (size_t)h * HD + 32 * s + 8 * grp);
                const float4 x0 = p[0], x1 = p[1];
                x[0] = to_h(x0.x * qsc); x[1] = to_h(x0.y * qsc); x[2] = to_h(x0.z * qsc); x[3] = to_h(x0.w * qsc);
                x[4] = to_h(x1.x * qsc); x[5] = to_h(x1.y * qsc); x[6] = to_h(x1.z * qsc); x[7] = to_h(x1.w * qsc);
            }
            qb[u][s] = x;
        }
    }

    floatx4 o[NT][NQT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int u = 0; u < NQT; ++u) o[t][u] = zero_f4();
    float m[NQT], l[NQT], lim[NQT];
#pragma unroll
    for (int u = 0; u < NQT; ++u) {
        m[u] = ninf();
        l[u] = 0.0f;
        const int r = p0 + 16 * u + col;
        lim[u] = (float)(a.causal ? min(a.past + r, ktot - 1) : ktot - 1);
    }
    const float sl2 = (a.scale_q ? 1.0f : a.scale) * LLMTIE_LOG2E;

    St st;
    if (kend > 0) load_tile(0, st);
    for (int kv0 = 0; kv0 < kend; kv0 += KT) {
        __syncthreads();  // previous tile fully consumed
        store_tile(kv0, st);
        __syncthreads();
        if (kv0 + KT < kend) load_tile(kv0 + KT, st);
        if (kv0 > wlim) continue;

        // S^T for the 64 keys: sc[hf][T][u], lane holds keys 32hf + 8grp + 4T + r.
        floatx4 sc[2][2][NQT];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int T = 0; T < 2; ++T) {
#pragma unroll
                for (int u = 0; u < NQT; ++u) sc[hf][T][u] = zero_f4();
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    const half8 af = kfrag(hf, T, s);
#pragma unroll
                    for (int u = 0; u < NQT; ++u) sc[hf][T][u] = mfma16(af, qb[u][s], sc[hf][T][u]);
                }
            }

        // Online softmax per query tile.
        half8 pb[2][NQT];
#pragma unroll
        for (int u = 0; u < NQT; ++u) {
            float mx = ninf();
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int T = 0; T < 2; ++T)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int key = kv0 + 32 * hf + 8 * grp + 4 * T + r;
                        const float s = (float)key <= lim[u] ? sc[hf][T][u][r] * sl2 : ninf();
                        sc[hf][T][u][r] = s;
                        mx = fmaxf(mx, s);
                    }
            mx = max4grp(mx);
            const float mn = fmaxf(m[u], mx);
            // A row whose every key so far is masked keeps m = -inf; its
            // factor and probabilities are then 0, never NaN.
            const float fac = mn == ninf() ? 1.0f : ex2(m[u] - mn);
            const float msub = mn == ninf() ? 0.0f : mn;
            m[u] = mn;
            float ps = 0.0f;
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                half8 p;
#pragma unroll
                for (int T = 0; T < 2; ++T)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float e = ex2(sc[hf][T][u][r] - msub);
                        ps += e;
                        p[4 * T + r] = to_h(e);
                    }
                pb[hf][u] = p;
            }
            l[u] = l[u] * fac + ps;
#pragma unroll
            for (int t = 0; t < NT; ++t) o[t][u] *= fac;
        }

        // O^T += V^T P^T.
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const half8 af = vfrag(hf, t);
#pragma unroll
                for (int u = 0; u < NQT; ++u) o[t][u] = mfma16(af, pb[hf][u], o[t][u]);
            }
    }

    // O / l, stored: lane writes dims 16t + 4grp + 0..3 of query p0 + 16u + col.
#pragma unroll
    for (int u = 0; u < NQT; ++u) {
        const float lt = sum4grp(l[u]);
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        const int r = p0 + 16 * u + col;
        if (r >= a.tq) continue;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const size_t off = (size_t)r * a.os + (size_t)h * HD + 16 * t + 4 * grp;
            if constexpr (KIND == PF_ROWS) {
                half4 y;
#pragma unroll
                for (int i = 0; i < 4; ++i) y[i] = to_h(o[t][u][i] * inv);
                *reinterpret_cast<half4*>(reinterpret_cast<half_t*>(a.out) + off) = y;
            } else {
                float4 y = make_float4(o[t][u][0] * inv, o[t][u][1] * inv, o[t][u][2] * inv, o[t][u][3] * inv);
                *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + off) = y;
            }
        }
    }
}


// ------------------------------------------------------------------------
// The f16-cache fast path (PF_F16 and PF_T16). Same work decomposition and
// arithmetic as flash_prefill_kernel, with the K/V tiles moved straight from
// global memory into LDS by global_load_lds_dwordx4 / buffer_load ... lds
// (no staging registers, no LDS store instructions), double-buffered with
// one barrier per tile, and the causal/tail mask applied only to the tiles
// that need it.
//
// LDS tile = the 64 keys' K fragments then V fragments, each fragment 64
// lanes x 16 bytes in exactly the order the MFMA A-operand reads take them
// (the tiled cache's fragment order): K fragment (half, T, s) holds, in lane
// l, key 32*half + 8*(col/4) + 4T + col%4, dims 32s + 8grp .. +7; V fragment
// (half, t) holds dim 16t + col, keys 32*half + 8grp .. +7. A tiled-cache
// tile is therefore two blocks copied verbatim, and the fragment reads are
// lane-contiguous and conflict-free. A reference-layout tile is held in
// line order instead (below).
//
// Keys past the cache's live ones: K rows are clamped to the last live row
// (their scores are masked); V chunks past ktot may hold anything, so in the
// one tile that reaches past ktot they are zeroed in LDS before use.
//
// The reference layout (PF_F16) is held in line order (lineorder.h): a
// fragment gathered straight from it would touch 16 lines, half of each, and
// a compute unit's rate of line requests would set the time to a tile (C3 at
// 512 rows: 17.1 us against 13.5 for the same tile from the tiled cache).
// W: waves per workgroup, 4, or 8 for the encoder rows (NQT = 1: the tile
// staging per query row of two query tiles per wave, at two waves per SIMD).
// Where the staged stacked-rows V tile keeps MFMA operand lane `ln` of dim
// tile t's fragment (a bijection of the 64 chunks for each t; the fragment
// read inverts nothing, it reads chunk rows_chunk(lane, t)). Writers put 2 (VR
// keys x 2 bytes) of a chunk's 16 bytes per lane.
//   VR = 2: chunk low nibble = 4 ((ln ^ t) & 3) + ((ln >> 2) & 3), i.e. the
//     two 2-bit fields of ln's low nibble swapped, the dim field XOR t. A
//     write instruction (fixed dim offset e, so ln & 3 = e) has its lanes at
//     ln = 4 r + e + 16 K over r, t and four key pairs (the 4-byte word of
//     the chunk): the chunk's low nibble 4 (e ^ t) + r is distinct over all
//     (r, t), and its low three bits over (r, t & 1) - the 64 lanes on 64
//     banks, each 32-lane half on 32.
//   VR = 4: ln ^ t (the low two bits XOR the dim tile).
template <int VR>
__device__ __forceinline__ int rows_chunk(int ln, int t) {
    if constexpr (VR == 2) return (ln & ~15) | (((ln ^ t) & 3) << 2) | ((ln >> 2) & 3);
    else return ln ^ (t & 3);
}

// A row's reference max before it has one: finite, so P = 2^(score * sl2 -
// m) of any live key overflows to +inf (and moves m), while masked keys
// (-inf) still give 0 and a row with no live key yet keeps it.
constexpr float PF_NOREF = -1e30f;
// The online softmax of query tile u over one 64-key tile, in log2 units:
// lane (col, grp) holds row 16u + col's scores of keys 32 hf + 8 grp + 4 T + r.
// P = 2^(score * sl2 - m) is formed against a reference max m that moves
// only when it must; O and l carry the same factor 2^-m, so O / l does not
// depend on where m sits. The probabilities are formed against the current
// m first; only when some lane's sum exceeds 2^15 (a score more than ~15
// above m, a row's first live key, or a NaN) does the wave take the tile's
// max, move m, rescale O and l and form them again. So every P is at most
// 2^15, inside f16 at full relative precision, m never exceeds the row's
// running max (no P is smaller than 2^(score - running max)), and the
// tile's max (16 maxima and a 4-lane reduction per row) is taken only on the
// rare tiles that move m.
template <bool MASK, int NT, int NQT>
__device__ __forceinline__ void softmax_tile(floatx4 (&sc)[2][2][NQT], int u, int kv0, int grp, int ilim,
                                             float sl2, float& m, float& l, floatx4 (&o)[NT][NQT],
                                             half8 (&pb)[2][NQT]) {
    if constexpr (MASK) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int T = 0; T < 2; ++T)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = kv0 + 32 * hf + 8 * grp + 4 * T + r;
                    sc[hf][T][u][r] = key <= ilim ? sc[hf][T][u][r] : ninf();
                }
    }
    auto form = [&]() __attribute__((always_inline)) {
        float ps = 0.0f;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            half8 p;
#pragma unroll
            for (int T = 0; T < 2; ++T)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float e = ex2(__builtin_fmaf(sc[hf][T][u][r], sl2, -m));
                    ps = (hf | T | r) ? ps + e : e;
                    p[4 * T + r] = to_h(e);
                }
            pb[hf][u] = p;
        }
        return ps;
    };
    float ps = form();
    if (__any(!(ps <= 32768.0f))) {
        float mx = ninf();
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int T = 0; T < 2; ++T)
#pragma unroll
                for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sc[hf][T][u][r]);
        const float mn = fmaxf(m, max4grp(mx) * sl2);
        const float fac = ex2(m - mn);
        m = mn;
        l *= fac;
#pragma unroll
        for (int t = 0; t < NT; ++t) o[t][u] *= fac;
        ps = form();
    }
    l += ps;
}

// Stores the context rows row0 .. row0 + 15 of head h (query tile u of the
// wave; rows >= tq skipped) in line order: the wave's O / l goes through its
// private LDS region R (16 x HD floats, a row's 16-byte chunk c at position
// c ^ (row & 15), so both the fragment-order writes and the row-order reads
// hit 16 different bank groups per 16 lanes), and each store instruction
// then writes whole lines (LPR lanes a row) instead of 16 rows' half lines
// (C3 at 512 rows 13.43 -> 13.31 us, at 128 rows 6.28 -> 6.16 us).
template <int HD, int NQT>
__device__ __forceinline__ void store_ctx16(float* R, const floatx4 (&o)[HD / 16][NQT], int u, float inv, int lane,
                                            const PrefillArgs& a, int row0, int h) {
    constexpr int NT = HD / 16, LPR = HD / 4, RPI = 64 / LPR;
    const int col = lane & 15, grp = lane >> 4;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float4 y = make_float4(o[t][u][0] * inv, o[t][u][1] * inv, o[t][u][2] * inv, o[t][u][3] * inv);
        *reinterpret_cast<float4*>(R + col * HD + 4 * ((4 * t + grp) ^ col)) = y;
    }
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int row = i * RPI + lane / LPR, c = lane % LPR;
        const float4 x = *reinterpret_cast<const float4*>(R + row * HD + 4 * (c ^ (row & 15)));
        if (row0 + row < a.tq) {
            const size_t off = (size_t)(row0 + row) * a.os + (size_t)h * HD + 4 * c;
            if (a.out_f16) {
                half4 y;
                y[0] = to_h(x.x); y[1] = to_h(x.y); y[2] = to_h(x.z); y[3] = to_h(x.w);
                *reinterpret_cast<half4*>(reinterpret_cast<half_t*>(a.out) + off) = y;
            } else {
                *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + off) = x;
            }
        }
    }
}

template <int HD, int KIND, int NQT, int W, bool QL>
__global__ __launch_bounds__(W * LLMTIE_WAVE, 8 / W) void flash_fwd_kernel(PrefillArgs a) {
    static_assert(W == PW || (W == 8 && KIND == PF_ROWS), "eight waves: encoder rows only");
    constexpr int TW = W * LLMTIE_WAVE;
    static_assert(KIND == PF_F16 || KIND == PF_T16 || KIND == PF_F32 || KIND == PF_ROWS, "unknown source");
    // f32 sources (the f32 cache, the stacked encoder rows) are staged through
    // registers: loaded as f32, rounded to f16 and written to LDS in the same
    // fragment order the direct-to-LDS kinds produce.
    constexpr bool STAGED = KIND == PF_F32 || KIND == PF_ROWS;
    constexpr int NS = HD / 32;
    constexpr int NT = HD / 16;
    constexpr int QPW = 16 * NQT;
    constexpr int KF = 4 * NS;          // K fragments per tile
    constexpr int VF = 2 * NT;          // V fragments per tile
    constexpr int FH = 64 * 8;          // halves per fragment
    constexpr int NF = (KF + VF) / W;  // fragments each wave loads per tile
    static_assert((KF + VF) % W == 0, "fragments split evenly over the waves");
    __shared__ __attribute__((aligned(16))) half_t t0[(KF + VF) * FH];
    __shared__ __attribute__((aligned(16))) half_t t1[(KF + VF) * FH];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int gb = a.gb;
    const int pb = QPW * (W / gb);
    const int group = a.heads / a.kv_heads;
    int rb = blockIdx.x, gy = blockIdx.y;
    if (a.xcd) {
        const int item = (int)(blockIdx.x % 8) * a.grid8 + (int)(blockIdx.x / 8);
        gy = item / a.nrb;
        rb = item % a.nrb;
    }
    // Causal: heaviest position blocks first.
    const int bx = a.causal ? a.nrb - 1 - rb : rb;
    const int h = gy * gb + wave % gb;
    const int kh = (gy * gb) / group;
    const int bp0 = bx * pb;
    const int p0 = bp0 + (wave / gb) * QPW;
    const int ktot = a.past + a.tq;
    const int kend = a.causal ? min(ktot, a.past + bp0 + pb) : ktot;
    // The last key any row of this wave sees, and the last key all of them see.
    const int wlim = a.causal ? min(a.past + p0 + QPW - 1, ktot - 1) : ktot - 1;
    const int wall = a.causal ? min(a.past + p0, ktot - 1) : ktot - 1;

    const half_t* kc = static_cast<const half_t*>(a.k);
    const size_t tblk = (size_t)kh * tiled_nblk(a.cap);
    const int lastb = (max(kend, 1) - 1) >> 5;
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.v), 0, (int)(uint32_t)a.v_bytes, 0x00020000);

    // Register staging (STAGED kinds). Fragment f = wave + W * i of a tile,
    // lane (col, grp): K fragment (half, T, s) is key 32*half + 8*(col/4) +
    // 4T + col%4, dims 32s + 8grp .. +7 (two float4 of one K row); V fragment
    // (half, t) is dim 16t + col, keys 32*half + 8grp .. +7 (two float4 of
    // one V^T row of the f32 cache, or one float from each of 8 stacked
    // rows). K rows past the live keys are clamped to the last live one (their
    // scores are masked); V entries past them are zero, so no tail pass is
    // needed. Every address stays below key ktot - 1 of its head.
    const float* kf32 = static_cast<const float*>(a.k);
    const float* vf32 = static_cast<const float*>(a.v);
    const size_t skb = KIND == PF_ROWS ? (size_t)kh * HD : (size_t)kh * a.cap * HD;  // K: head base
    const size_t skr = KIND == PF_ROWS ? (size_t)a.kvs : (size_t)HD;                 // K: row stride
    const size_t svb = KIND == PF_ROWS ? (size_t)kh * HD : (size_t)kh * HD * a.cap;  // V: head base
    const bool vvec = KIND == PF_F32 && a.cap % 4 == 0;  // V^T rows 16-byte aligned
    constexpr int NSR = STAGED ? NF : 1;
    // Staged tiles in flight: tile j's f32 loads are issued SPD periods
    // before it is written to LDS (the K/V rows come from L2 or the Infinity
    // Cache, whose latency is several tiles' compute at the encoder's
    // shape). SPD register sets rotate, so the period loop is unrolled by
    // SU = lcm(SPD, 2) (the two LDS buffers).
    constexpr int SPD = KIND == PF_ROWS ? LLMTIE_PF_SPD : 1;
    constexpr int SU = SPD % 2 == 0 ? SPD : 2 * SPD;
    float4 sr[SPD][NSR][2];
    // Stacked rows: V is [key][dim], so a thread takes 4 dims x VR keys
    // (one float4 from each of VR rows; 16 threads cover one 256-byte row
    // segment) instead of one fragment chunk, and writes each dim's VR keys
    // as one 2·VR-byte piece of a chunk. The V fragments are the wave's last
    // NF - KF / W staging slots.
    constexpr int KI = KF / W;         // staging slots holding K fragments
    constexpr int VR = 1024 / TW;      // rows V: keys per thread (4, or 2 at eight waves)
    static_assert(KIND != PF_ROWS || (HD == 64 && KF % W == 0 && 2 * (NF - KI) == VR), "rows: hd 64");
    // Rows V: thread takes dims 4*rdq .. +3 of keys kb .. kb + VR - 1. At VR
    // = 2 (eight waves) lane = (rdq & 3) + 4 kp + 16 (rdq >> 2) for key pair
    // kp: four consecutive lanes read one row's 64 contiguous bytes, and each
    // 32-lane half of a 4-byte LDS write covers 8 dims x 4 key pairs, which
    // the chunk swizzle (rows_chunk) puts on 32 distinct banks (64 for the
    // whole wave). (Key pair fastest, lane = kp + 4 rdq, was as free of bank
    // conflicts but scattered the row reads: C4 encoder 36.3 vs 34.0 us.)
    const int rdq = VR == 2 ? (tid & 3) + 4 * ((tid >> 4) & 3) : tid & 15;
    const int kb = VR == 2 ? VR * (((tid >> 2) & 3) + 4 * (tid >> 6)) : VR * (tid >> 4);
    auto stage_load = [&](auto set_tag, int kv0) __attribute__((always_inline)) {
        constexpr int SS = decltype(set_tag)::value;
        if constexpr (KIND == PF_ROWS) {
#pragma unroll
            for (int u = 0; u < VR; ++u) {
                const int key = kv0 + kb + u;
                const float4 x = *reinterpret_cast<const float4*>(vf32 + svb + (size_t)min(key, ktot - 1) * a.kvs +
                                                                  4 * rdq);
                sr[SS][KI + u / 2][u % 2] = x;  // zeroed past the keys when stored
            }
        }
        if constexpr (STAGED) {
#pragma unroll
            for (int i = 0; i < NF; ++i) {
                const int f = wave + W * i;
                if (KIND == PF_ROWS && i >= KI) continue;
                // Rows: the K fragments are the first KI = KF / W slots of
                // every wave, never a V one (so no dead V branch sits between
                // the loads and leaves their waits conservative).
                if (KIND == PF_ROWS || f < KF) {
                    const int hf = f / (2 * NS), T = (f / NS) & 1, s = f % NS;
                    const int key = min(kv0 + 32 * hf + 8 * (col >> 2) + 4 * T + (col & 3), ktot - 1);
                    const float4* p = reinterpret_cast<const float4*>(kf32 + skb + (size_t)key * skr + 32 * s + 8 * grp);
                    sr[SS][i][0] = p[0];
                    sr[SS][i][1] = p[1];
                } else if constexpr (KIND != PF_ROWS) {
                    const int fv = f - KF, hf = fv / NT, t = fv % NT;
                    const int d = 16 * t + col, k0 = kv0 + 32 * hf + 8 * grp;
                    float4 v0, v1;
                    if (vvec && k0 + 8 <= ktot) {
                        const float4* p = reinterpret_cast<const float4*>(vf32 + svb + (size_t)d * a.cap + k0);
                        v0 = p[0];
                        v1 = p[1];
                    } else {
                        float x[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            // Loaded unconditionally at the clamped key, then
                            // selected: a load under a lane-varying condition
                            // is waited for at the branch's end.
                            const int key = min(k0 + j, ktot - 1);
                            const float y = vf32[svb + (size_t)d * a.cap + key];
                            x[j] = k0 + j < ktot ? y : 0.0f;
                        }
                        v0 = make_float4(x[0], x[1], x[2], x[3]);
                        v1 = make_float4(x[4], x[5], x[6], x[7]);
                    }
                    sr[SS][i][0] = v0;
                    sr[SS][i][1] = v1;
                }
            }
        }
    };
    auto stage_store = [&](auto set_tag, half_t* dst, int kv0) __attribute__((always_inline)) {
        constexpr int SS = decltype(set_tag)::value;
        if constexpr (KIND == PF_ROWS) {
            // Dim 4*rdq + e, keys kb .. kb + VR - 1: V fragment (half, t) =
            // (kb / 32, dim / 16), lane (dim % 16) + 16 * ((kb / 8) % 4), halves kb % 8 ..
            typedef _Float16 hv __attribute__((ext_vector_type(VR)));
            float4 x[VR];
#pragma unroll
            for (int u = 0; u < VR; ++u) x[u] = sr[SS][KI + u / 2][u % 2];
            // Only the tile reaching past the keys has V rows to zero: a
            // wave-uniform branch, so full tiles convert with no per-key select.
            if (kv0 + KT > ktot) {
#pragma unroll
                for (int u = 0; u < VR; ++u)
                    if (kv0 + kb + u >= ktot) x[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int dd = 4 * rdq + e;
                hv y;
#pragma unroll
                for (int u = 0; u < VR; ++u) y[u] = to_h(e == 0 ? x[u].x : e == 1 ? x[u].y : e == 2 ? x[u].z : x[u].w);
                const int frag = KF + (kb >> 5) * NT + (dd >> 4);
                // The MFMA operand lane holding this dim and key group, moved
                // to the chunk rows_chunk gives it; the fragment read applies
                // the same map.
                const int ln = rows_chunk<VR>((dd & 15) + 16 * ((kb >> 3) & 3), dd >> 4);
                *reinterpret_cast<hv*>(dst + frag * FH + ln * 8 + (kb & 7)) = y;
            }
        }
        if constexpr (STAGED) {
#pragma unroll
            for (int i = 0; i < NF; ++i) {
                const int f = wave + W * i;
                if (KIND == PF_ROWS && i >= KI) continue;
                const float4 x0 = sr[SS][i][0], x1 = sr[SS][i][1];
                half8 y;
                y[0] = to_h(x0.x); y[1] = to_h(x0.y); y[2] = to_h(x0.z); y[3] = to_h(x0.w);
                y[4] = to_h(x1.x); y[5] = to_h(x1.y); y[6] = to_h(x1.z); y[7] = to_h(x1.w);
                reinterpret_cast<half8*>(dst + f * FH)[lane] = y;
            }
        }
    };

    auto issue = [&](int kv0, half_t* dst) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            const int f = wave + W * i;
            half_t* l = dst + f * FH;
            if constexpr (STAGED) {
                (void)l;
            } else if constexpr (KIND == PF_T16) {
                const int hf = f < KF ? f / (2 * NS) : (f - KF) / NT;
                const int b = min((kv0 >> 5) + hf, lastb);
                const int in = f < KF ? (f % (2 * NS)) * FH : 32 * HD + ((f - KF) % NT) * FH;
                __builtin_amdgcn_global_load_lds(kc + (tblk + b) * (64 * HD) + in + lane * 8, l, 16, 0, 0);
            } else {
                pfl_issue<HD, KF>(kc, rv, f, lane, (size_t)kh, (size_t)a.cap, kv0, ktot, l);
            }
        }
    };

    // Q as B operands: qb[u][s] holds dims 32s + 8grp + 0..7 of query p0 + 16u + col.
    // The first tile's loads go out before the query's (the query's first
    // use waits for every load issued before it, tile loads included: the
    // compiler does not count LDS-DMA loads in order).
    if constexpr (STAGED) {
        // Unconditional (rows past the keys are clamped to the last one), so
        // no branch leaves the compiler unsure how many loads are pending.
        if (kend > 0) static_for<SPD>([&](auto i) { stage_load(i, decltype(i)::value * KT); });
    } else {
        // A causal launch of at most one workgroup per compute unit is as
        // long as its heaviest blocks' tile chain: the light blocks (at most
        // half the heaviest's tiles) hold their first loads back ~0.85 us so
        // the heavy blocks' queries and first tiles meet less traffic.
        if (a.light_tiles > 0 && (kend + KT - 1) / KT <= a.light_tiles) __builtin_amdgcn_s_sleep(LLMTIE_PF_SLEEP);
        if (kend > 0) issue(0, t0);
    }
    const float qsc = a.scale_q ? a.scale : 1.0f;
    half8 qb[NQT][NS];
    if constexpr (QL) {
        // QL: the wave's query rows read in line order (each instruction 1
        // KB of whole rows: RPI rows of LPR lanes x 4 floats), scaled,
        // rounded to f16 and passed through this wave's part of buffer t1
        // (free until the second tile is issued, after the first barrier)
        // into fragment order. Read straight in fragment order, each
        // instruction touches 16 rows' lines, half of each, which a launch
        // of few workgroups (one per compute unit, or fewer) pays in its
        // time to first tile. In t1 a row's 16-byte chunk c sits at
        // position c ^ qsw(row), so a fragment read's 16 rows hit 16
        // different bank groups.
        constexpr int LPR = HD / 4, RPI = 64 / LPR, NI = QPW / RPI;
        static_assert(W * QPW * HD <= (KF + VF) * FH, "the queries fit buffer t1");
        auto qsw = [](int row) { return HD == 128 ? (row & 15) : ((row >> 1) & 7); };
        half_t* qs = t1 + wave * QPW * HD;
        float4 qx[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int r = min(p0 + i * RPI + lane / LPR, a.tq - 1);
            qx[i] = *reinterpret_cast<const float4*>(a.q + (size_t)r * a.qs + (size_t)h * HD + 4 * (lane % LPR));
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int row = i * RPI + lane / LPR;
            const float m = p0 + row < a.tq ? qsc : 0.0f;
            half4 y;
            y[0] = to_h(qx[i].x * m); y[1] = to_h(qx[i].y * m); y[2] = to_h(qx[i].z * m); y[3] = to_h(qx[i].w * m);
            const int c = (lane % LPR) >> 1;
            *reinterpret_cast<half4*>(qs + row * HD + (c ^ qsw(row)) * 8 + (lane & 1) * 4) = y;
        }
#pragma unroll
        for (int u = 0; u < NQT; ++u)
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const int row = 16 * u + col;
                qb[u][s] = *reinterpret_cast<const half8*>(qs + row * HD + ((4 * s + grp) ^ qsw(row)) * 8);
            }
    } else {
        float4 qx[NQT][NS][2];
#pragma unroll
        for (int u = 0; u < NQT; ++u) {
            const int r = min(p0 + 16 * u + col, a.tq - 1);
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const float4* p =
                    reinterpret_cast<const float4*>(a.q + (size_t)r * a.qs + (size_t)h * HD + 32 * s + 8 * grp);
                qx[u][s][0] = p[0];
                qx[u][s][1] = p[1];
            }
        }
#pragma unroll
        for (int u = 0; u < NQT; ++u) {
            const float m = p0 + 16 * u + col < a.tq ? qsc : 0.0f;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const float4 x0 = qx[u][s][0], x1 = qx[u][s][1];
                half8 x;
                x[0] = to_h(x0.x * m); x[1] = to_h(x0.y * m); x[2] = to_h(x0.z * m); x[3] = to_h(x0.w * m);
                x[4] = to_h(x1.x * m); x[5] = to_h(x1.y * m); x[6] = to_h(x1.z * m); x[7] = to_h(x1.w * m);
                qb[u][s] = x;
            }
        }
    }

    floatx4 o[NT][NQT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int u = 0; u < NQT; ++u) o[t][u] = zero_f4();
    float m[NQT], l[NQT];
    int ilim[NQT];
#pragma unroll
    for (int u = 0; u < NQT; ++u) {
        m[u] = PF_NOREF;
        l[u] = 0.0f;
        const int r = p0 + 16 * u + col;
        ilim[u] = a.causal ? min(a.past + r, ktot - 1) : ktot - 1;
    }
    const float sl2 = (a.scale_q ? 1.0f : a.scale) * LLMTIE_LOG2E;

    // One 64-key tile from LDS buffer `tb`; MASK: some key of it lies past
    // some row's limit.
    auto tile = [&](const half_t* tb, int kv0, auto mask_tag) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const half8* kf = reinterpret_cast<const half8*>(tb);
        const half8* vf = reinterpret_cast<const half8*>(tb + KF * FH);
        floatx4 sc[2][2][NQT];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int T = 0; T < 2; ++T)
#pragma unroll
                for (int u = 0; u < NQT; ++u) sc[hf][T][u] = zero_f4();
        // Dims outermost: 4 * NQT independent accumulators between two
        // products into the same one (each still sums its dims in order).
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int T = 0; T < 2; ++T) {
                    const int k = 32 * hf + 8 * (col >> 2) + 4 * T + (col & 3);
                    const half8 af = kf[KIND == PF_F16 ? pfl_kslot<HD>(k, 4 * s + grp) : ((hf * 2 + T) * NS + s) * 64 + lane];
#pragma unroll
                    for (int u = 0; u < NQT; ++u) sc[hf][T][u] = mfma16(af, qb[u][s], sc[hf][T][u]);
                }
        // Software pipeline: PD fragment reads ahead of the MFMAs using them.
        {
            constexpr int NR = 4 * NS, PD = LLMTIE_PF_PD < NR ? LLMTIE_PF_PD : NR;
            __builtin_amdgcn_sched_group_barrier(0x100, PD, 0);
#pragma unroll
            for (int i2 = 0; i2 < NR - PD; ++i2) {
                __builtin_amdgcn_sched_group_barrier(0x008, NQT, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NQT * PD, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        half8 pb[2][NQT];
#pragma unroll
        for (int u = 0; u < NQT; ++u) softmax_tile<MASK>(sc, u, kv0, grp, ilim[u], sl2, m[u], l[u], o, pb);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                // Rows: V chunks are swizzled by the dim tile (stage_store);
                // the reference layout is in line order.
                const half8 af = vf[KIND == PF_F16 ? pfl_vslot(16 * t + col, 4 * hf + grp)
                                                   : (hf * NT + t) * 64 +
                                                         (KIND == PF_ROWS ? rows_chunk<1024 / TW>(lane, t) : lane)];
#pragma unroll
                for (int u = 0; u < NQT; ++u) o[t][u] = mfma16(af, pb[hf][u], o[t][u]);
            }
        {
            constexpr int NR = 2 * NT, PD = LLMTIE_PF_PD < NR ? LLMTIE_PF_PD : NR;
            __builtin_amdgcn_sched_group_barrier(0x100, PD, 0);
#pragma unroll
            for (int i2 = 0; i2 < NR - PD; ++i2) {
                __builtin_amdgcn_sched_group_barrier(0x008, NQT, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NQT * PD, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // Zero the V entries of keys >= ktot in a tile that reaches past ktot.
    auto zero_tail = [&](half_t* tb, int kv0) __attribute__((always_inline)) {
        pf_zero_tail<HD, KIND == PF_F16>(reinterpret_cast<half8*>(tb + KF * FH), kv0, ktot, tid, TW);
    };
    auto step = [&](half_t* cur, half_t* nxt, int kv0) __attribute__((always_inline)) {
        __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of `cur` have landed
        __syncthreads();                 // ... and every wave's; `nxt` is free
        if (kv0 + KT < kend) issue(kv0 + KT, nxt);
        if (kv0 + KT > ktot) {
            zero_tail(cur, kv0);
            __syncthreads();
        }
        if (kv0 > wlim) return;
        if (kv0 + KT - 1 > wall)
            tile(cur, kv0, std::true_type{});
        else
            tile(cur, kv0, std::false_type{});
    };

    // Staged kinds: tile j is in LDS buffer `cur` when the barrier passes;
    // tile j + SPD's f32 loads go out into the register set tile j left
    // (written to LDS at the end of the period before), tile j is computed,
    // then tile j + 1 (loaded SPD - 1 periods ago) is rounded and written to
    // `nxt`, which every wave finished reading before that barrier.
    auto step_staged = [&](auto jj_tag, half_t* cur, half_t* nxt, int kv0) __attribute__((always_inline)) {
        constexpr int JJ = decltype(jj_tag)::value;
        __syncthreads();
        stage_load(std::integral_constant<int, JJ % SPD>{}, kv0 + SPD * KT);
        __builtin_amdgcn_sched_barrier(0);
        if (kv0 <= wlim && kv0 < kend) {
            if (kv0 + KT - 1 > wall)
                tile(cur, kv0, std::true_type{});
            else
                tile(cur, kv0, std::false_type{});
        }
        __builtin_amdgcn_sched_barrier(0);
        stage_store(std::integral_constant<int, (JJ + 1) % SPD>{}, nxt, kv0 + KT);
    };
    if constexpr (STAGED) {
        if (kend > 0) stage_store(std::integral_constant<int, 0>{}, t0, 0);
        // Whole rounds of SU periods; the periods past the last tile only
        // load clamped rows and write a tile nobody reads.
        for (int kv0 = 0; kv0 < kend; kv0 += SU * KT)
            static_for<SU>([&](auto jj) {
                constexpr int JJ = decltype(jj)::value;
                step_staged(jj, JJ % 2 ? t1 : t0, JJ % 2 ? t0 : t1, kv0 + JJ * KT);
            });
    } else {
        for (int kv0 = 0; kv0 < kend; kv0 += 2 * KT) {
            step(t0, t1, kv0);
            if (kv0 + KT < kend) step(t1, t0, kv0 + KT);
        }
    }

    if constexpr (!STAGED) {
        // O / l stored in line order (store_ctx16) through the tile buffer
        // that does not hold the last tile: every wave finished reading it
        // before the last tile's barrier, which this wave has passed, and
        // no later tile is issued into it. Wave w's region: 16 x HD floats.
        static_assert(W * 16 * HD * 4 <= (KF + VF) * FH * 2, "the waves' regions fit one tile buffer");
        const int nt = (kend + KT - 1) / KT;
        float* R = reinterpret_cast<float*>(nt % 2 ? t1 : t0) + wave * 16 * HD;
#pragma unroll
        for (int u = 0; u < NQT; ++u) {
            const float lt = sum4grp(l[u]);
            store_ctx16<HD, NQT>(R, o, u, lt > 0.0f ? 1.0f / lt : 0.0f, lane, a, p0 + 16 * u, h);
        }
        return;
    }
    // Staged kinds (their last period writes the other buffer): O / l
    // stored straight from the fragments; lane writes dims 16t + 4grp + 0..3 of query p0 + 16u + col.
#pragma unroll
    for (int u = 0; u < NQT; ++u) {
        const float lt = sum4grp(l[u]);
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        const int r = p0 + 16 * u + col;
        if (r >= a.tq) continue;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const size_t off = (size_t)r * a.os + (size_t)h * HD + 16 * t + 4 * grp;
            if (a.out_f16) {
                half4 y;
#pragma unroll
                for (int i = 0; i < 4; ++i) y[i] = to_h(o[t][u][i] * inv);
                *reinterpret_cast<half4*>(reinterpret_cast<half_t*>(a.out) + off) = y;
            } else {
                float4 y = make_float4(o[t][u][0] * inv, o[t][u][1] * inv, o[t][u][2] * inv, o[t][u][3] * inv);
                *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + off) = y;
            }
        }
    }
}

// ------------------------------------------------------------------------
// Long prefills: the f16-cache kernel in "ping-pong" form. A workgroup is
// eight waves in two groups of four (A: waves 0-3, B: waves 4-7); waves w and
// w + 4 share a SIMD. Both groups hold 32 query rows per wave (two 16-row
// tiles) and share each 64-key K/V tile in LDS. Per tile a wave's work is
// S = K Q^T (MFMA), the softmax (VALU) and O += V^T P^T (MFMA). Between two
// workgroup barriers (one tile period) group A computes PV(q - 1), S(q) and
// then softmax(q), group B softmax(q - 1) and then PV(q - 1), S(q), so the
// two waves of each SIMD start every period in opposite units and the
// softmax of one overlaps the MFMAs of the other (in the four-wave kernel
// the two waves of a SIMD come from different workgroups, drift into the
// same phase, and VALU issues beside MFMAs in only ~22 % of MFMA cycles).
// The arithmetic per row is the four-wave kernel's, in the same order, so
// the results are bit-identical. (A stricter version, a barrier at every
// phase change, raised the co-issue by half but lost more to the barrier
// waits of a whole compute unit: C3 at 8192 rows 634 vs 612 µs.)
//
// Tiles rotate through three LDS buffers: period q reads K_q and V_(q-1);
// tile q + 1 is issued at the start of period q into the buffer of tile
// q - 2 and waited for at the end of period q.
constexpr int PPW = 8;  // waves of a ping-pong workgroup

template <int HD, int KIND>
__global__ __launch_bounds__(PPW * LLMTIE_WAVE, 1) void flash_pp_kernel(PrefillArgs a) {
    static_assert(KIND == PF_F16 || KIND == PF_T16, "f16 caches");
    constexpr int NQT = 2;
    constexpr int NS = HD / 32;
    constexpr int NT = HD / 16;
    constexpr int QPW = 16 * NQT;
    constexpr int KF = 4 * NS;
    constexpr int VF = 2 * NT;
    constexpr int FH = 64 * 8;
    constexpr int NF = (KF + VF) / PPW;  // fragments each wave loads per tile
    constexpr int TPW = PPW * LLMTIE_WAVE;
    static_assert((KF + VF) % PPW == 0, "fragments split evenly over the waves");
    __shared__ __attribute__((aligned(16))) half_t tbuf[3][(KF + VF) * FH];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int gi = wave >> 2;  // 0: group A, 1: group B
    const int wl = wave & 3;
    const int gb = a.gb;
    const int gpr = QPW * (4 / gb);  // rows of one group
    const int pb = 2 * gpr;          // rows of the workgroup
    const int group = a.heads / a.kv_heads;
    int rb = blockIdx.x, gy = blockIdx.y;
    if (a.xcd) {
        const int item = (int)(blockIdx.x % 8) * a.grid8 + (int)(blockIdx.x / 8);
        gy = item / a.nrb;
        rb = item % a.nrb;
    }
    const int bx = a.causal ? a.nrb - 1 - rb : rb;
    const int h = gy * gb + wl % gb;
    const int kh = (gy * gb) / group;
    const int bp0 = bx * pb;
    const int p0 = bp0 + gi * gpr + (wl / gb) * QPW;
    const int ktot = a.past + a.tq;
    const int kend = a.causal ? min(ktot, a.past + bp0 + pb) : ktot;
    const int wlim = a.causal ? min(a.past + p0 + QPW - 1, ktot - 1) : ktot - 1;
    const int wall = a.causal ? min(a.past + p0, ktot - 1) : ktot - 1;
    const int ntile = (kend + KT - 1) / KT;

    const half_t* kc = static_cast<const half_t*>(a.k);
    const size_t tblk = (size_t)kh * tiled_nblk(a.cap);
    const int lastb = (max(kend, 1) - 1) >> 5;
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.v), 0, (int)(uint32_t)a.v_bytes, 0x00020000);

    auto issue = [&](int kv0, half_t* dst) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            const int f = wave + PPW * i;
            half_t* l = dst + f * FH;
            if constexpr (KIND == PF_T16) {
                const int hf = f < KF ? f / (2 * NS) : (f - KF) / NT;
                const int b = min((kv0 >> 5) + hf, lastb);
                const int in = f < KF ? (f % (2 * NS)) * FH : 32 * HD + ((f - KF) % NT) * FH;
                __builtin_amdgcn_global_load_lds(kc + (tblk + b) * (64 * HD) + in + lane * 8, l, 16, 0, 0);
            } else {
                pfl_issue<HD, KF>(kc, rv, f, lane, (size_t)kh, (size_t)a.cap, kv0, ktot, l);
            }
        }
    };
    auto zero_tail = [&](half_t* tb, int kv0) __attribute__((always_inline)) {
        pf_zero_tail<HD, KIND == PF_F16>(reinterpret_cast<half8*>(tb + KF * FH), kv0, ktot, tid, TPW);
    };

    // The first three tiles go out before the queries are read.
#pragma unroll
    for (int j = 0; j < 3; ++j)
        if (j < ntile) issue(j * KT, tbuf[j]);
    const float qsc = a.scale_q ? a.scale : 1.0f;
    half8 qb[NQT][NS];
#pragma unroll
    for (int u = 0; u < NQT; ++u) {
        const int r = min(p0 + 16 * u + col, a.tq - 1);
        const float m = p0 + 16 * u + col < a.tq ? qsc : 0.0f;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const float4* p = reinterpret_cast<const float4*>(a.q + (size_t)r * a.qs + (size_t)h * HD + 32 * s + 8 * grp);
            const float4 x0 = p[0], x1 = p[1];
            half8 x;
            x[0] = to_h(x0.x * m); x[1] = to_h(x0.y * m); x[2] = to_h(x0.z * m); x[3] = to_h(x0.w * m);
            x[4] = to_h(x1.x * m); x[5] = to_h(x1.y * m); x[6] = to_h(x1.z * m); x[7] = to_h(x1.w * m);
            qb[u][s] = x;
        }
    }
    floatx4 o[NT][NQT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int u = 0; u < NQT; ++u) o[t][u] = zero_f4();
    float m[NQT], l[NQT];
    int ilim[NQT];
#pragma unroll
    for (int u = 0; u < NQT; ++u) {
        m[u] = PF_NOREF;
        l[u] = 0.0f;
        const int r = p0 + 16 * u + col;
        ilim[u] = a.causal ? min(a.past + r, ktot - 1) : ktot - 1;
    }
    const float sl2 = (a.scale_q ? 1.0f : a.scale) * LLMTIE_LOG2E;
    floatx4 sc[2][2][NQT];
    half8 pb2[2][NQT];

    auto scores = [&](const half_t* tb) __attribute__((always_inline)) {
        const half8* kf = reinterpret_cast<const half8*>(tb);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int T = 0; T < 2; ++T)
#pragma unroll
                for (int u = 0; u < NQT; ++u) sc[hf][T][u] = zero_f4();
        // Dims outermost: 4 * NQT independent accumulators between two
        // products into the same one (each still sums its dims in order).
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int T = 0; T < 2; ++T) {
                    const int k = 32 * hf + 8 * (col >> 2) + 4 * T + (col & 3);
                    const half8 af = kf[KIND == PF_F16 ? pfl_kslot<HD>(k, 4 * s + grp) : ((hf * 2 + T) * NS + s) * 64 + lane];
#pragma unroll
                    for (int u = 0; u < NQT; ++u) sc[hf][T][u] = mfma16(af, qb[u][s], sc[hf][T][u]);
                }
        {
            constexpr int NR = 4 * NS, PD = LLMTIE_PF_PD < NR ? LLMTIE_PF_PD : NR;
            __builtin_amdgcn_sched_group_barrier(0x100, PD, 0);
#pragma unroll
            for (int i2 = 0; i2 < NR - PD; ++i2) {
                __builtin_amdgcn_sched_group_barrier(0x008, NQT, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NQT * PD, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    auto values = [&](const half_t* tb) __attribute__((always_inline)) {
        const half8* vf = reinterpret_cast<const half8*>(tb + KF * FH);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const half8 af = vf[KIND == PF_F16 ? pfl_vslot(16 * t + col, 4 * hf + grp) : (hf * NT + t) * 64 + lane];
#pragma unroll
                for (int u = 0; u < NQT; ++u) o[t][u] = mfma16(af, pb2[hf][u], o[t][u]);
            }
        {
            constexpr int NR = 2 * NT, PD = LLMTIE_PF_PD < NR ? LLMTIE_PF_PD : NR;
            __builtin_amdgcn_sched_group_barrier(0x100, PD, 0);
#pragma unroll
            for (int i2 = 0; i2 < NR - PD; ++i2) {
                __builtin_amdgcn_sched_group_barrier(0x008, NQT, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NQT * PD, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    auto softmax = [&](int kv0, auto mask_tag) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
        for (int u = 0; u < NQT; ++u) softmax_tile<MASK>(sc, u, kv0, grp, ilim[u], sl2, m[u], l[u], o, pb2);
    };

    if (ntile > 0) {
        __builtin_amdgcn_s_waitcnt(0);
        if (KT > ktot) zero_tail(tbuf[0], 0);
    }
    __syncthreads();
    auto smax = [&](int j) __attribute__((always_inline)) {
        if (j * KT + KT - 1 > wall)
            softmax(j * KT, std::true_type{});
        else
            softmax(j * KT, std::false_type{});
    };
    {
        // One barrier per tile period q: K_q and V_(q-1) are read. Group A
        // computes PV(q - 1), S(q) then softmax(q); group B softmax(q - 1)
        // then PV(q - 1), S(q): the two waves of a SIMD start each period in
        // opposite units. Tile q + 1 is issued at the start of period q into
        // the buffer of tile q - 2 (last read in period q - 1) and waited for
        // at its end; V past ktot of tile q is zeroed in period q, before
        // period q + 1 reads it.
        for (int q = 0; q <= ntile; ++q) {
            if (q >= 2 && q + 1 < ntile) issue((q + 1) * KT, tbuf[(q + 1) % 3]);
            if (q >= 1 && q < ntile && q * KT + KT > ktot) zero_tail(tbuf[q % 3], q * KT);
            if (gi == 0) {
                if (q >= 1 && (q - 1) * KT <= wlim) values(tbuf[(q - 1) % 3]);
                if (q < ntile && q * KT <= wlim) {
                    scores(tbuf[q % 3]);
                    smax(q);
                }
            } else {
                if (q >= 1 && (q - 1) * KT <= wlim) {
                    smax(q - 1);
                    values(tbuf[(q - 1) % 3]);
                }
                if (q < ntile && q * KT <= wlim) scores(tbuf[q % 3]);
            }
            __builtin_amdgcn_s_waitcnt(0);  // the tile issued at the start of this period
            __syncthreads();
        }
    }
#pragma unroll
    for (int u = 0; u < NQT; ++u) {
        const float lt = sum4grp(l[u]);
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        const int r = p0 + 16 * u + col;
        if (r >= a.tq) continue;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const size_t off = (size_t)r * a.os + (size_t)h * HD + 16 * t + 4 * grp;
            if (a.out_f16) {
                half4 y;
#pragma unroll
                for (int k = 0; k < 4; ++k) y[k] = to_h(o[t][u][k] * inv);
                *reinterpret_cast<half4*>(reinterpret_cast<half_t*>(a.out) + off) = y;
            } else {
                float4 y = make_float4(o[t][u][0] * inv, o[t][u][1] * inv, o[t][u][2] * inv, o[t][u][3] * inv);
                *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + off) = y;
            }
        }
    }
}

hipError_t launch_prefill(int hd, int kind, int nqt, const PrefillArgs& a, hipStream_t st, int waves) {
    // Eight-wave workgroups: the encoder rows at one query tile per wave only.
    const bool w8 = waves == 8 && hd == 64 && kind == PF_ROWS && nqt == 1;
    const int pb = 16 * nqt * ((w8 ? 8 : PW) / a.gb);
    dim3 grid((a.tq + pb - 1) / pb, a.heads / a.gb), block(w8 ? 8 * LLMTIE_WAVE : PT);
#define L(HD, KIND, NQ)                                                                      \
    if (hd == HD && kind == KIND && nqt == NQ) {                                             \
        hipLaunchKernelGGL((flash_prefill_kernel<HD, KIND, NQ>), grid, block, 0, st, a);     \
        return hipGetLastError();                                                            \
    }
#define LK(HD, KIND) L(HD, KIND, 1) L(HD, KIND, 2) L(HD, KIND, 4)
    // The f16 caches take the direct-to-LDS kernel when the V cache is
    // addressable by a 32-bit buffer offset (always, for the tiled cache).
    // (It keeps the raw-score max, so it needs a positive score scale.)
    // The f32 sources take it through register staging when K and V are
    // 16-byte aligned (rows: a row stride of whole float4s).
    const bool al16 = ((reinterpret_cast<uintptr_t>(a.k) | reinterpret_cast<uintptr_t>(a.v)) & 15) == 0;
    const bool f32ok = (kind == PF_F32 && al16) || (kind == PF_ROWS && al16 && a.kvs % 4 == 0);
    const bool fast = (kind == PF_T16 || (kind == PF_F16 && a.v_bytes <= 0xffffffffull) || f32ok) &&
                      (a.scale_q || a.scale > 0.0f) && !getenv("LLMTIE_PREFILL_STAGED");
    if (w8 && !fast) return launch_prefill(hd, kind, nqt, a, st, 4);
    // Long prefills of an f16 cache: the ping-pong kernel, once its 64-row
    // workgroups still fill the chip (LLMTIE_PREFILL_PP=0 turns it off, =1
    // forces it where it applies).
    const char* ppe = getenv("LLMTIE_PREFILL_PP");
    const int pp_rows = 2 * 32 * (4 / a.gb);
    const unsigned pp_items = (unsigned)((a.tq + pp_rows - 1) / pp_rows) * (unsigned)(a.heads / a.gb);
    const bool pp = fast && (kind == PF_T16 || kind == PF_F16) && !(ppe && !atoi(ppe)) &&
                    ((ppe && atoi(ppe)) || pp_items >= 1024);
    if (pp) {
        PrefillArgs b = a;
        b.nrb = (a.tq + pp_rows - 1) / pp_rows;
        b.xcd = pp_items % 8 == 0 && !(getenv("LLMTIE_PREFILL_XCD") && !atoi(getenv("LLMTIE_PREFILL_XCD")));
        b.grid8 = (int)(pp_items / 8);
        const dim3 g = b.xcd ? dim3(pp_items) : dim3(b.nrb, a.heads / a.gb);
        const dim3 blk(PPW * LLMTIE_WAVE);
#define PPL(HD, KIND)                                                          \
    if (hd == HD && kind == KIND) {                                             \
        hipLaunchKernelGGL((flash_pp_kernel<HD, KIND>), g, blk, 0, st, b);      \
        return hipGetLastError();                                               \
    }
        PPL(64, PF_F16) PPL(128, PF_F16) PPL(64, PF_T16) PPL(128, PF_T16)
#undef PPL
    }
    if (fast) {
        PrefillArgs b = a;
        b.nrb = (int)grid.x;
        const unsigned items = grid.x * grid.y;
        b.xcd = items % 8 == 0 && !(getenv("LLMTIE_PREFILL_XCD") && !atoi(getenv("LLMTIE_PREFILL_XCD")));
        b.grid8 = (int)(items / 8);
        const int heavy = (a.past + a.tq + KT - 1) / KT;
        b.light_tiles = a.causal && !w8 && (int)items <= a.cus && heavy >= 6 && LLMTIE_PF_SLEEP > 0 ? heavy / 2 : 0;
        const dim3 g = b.xcd ? dim3(items) : grid;
        // Line-order query loads (QL) where they pay: f16-cache launches of
        // at most half a workgroup per compute unit (C3 at 128 rows 6.52 ->
        // 6.30 us). At one workgroup per compute unit (C3 at 512 rows) they
        // cost 0.2 us, and the encoder rows measured within noise.
        const bool ql = (int)items * 2 <= a.cus && !getenv("LLMTIE_PREFILL_NOQL");
        if (w8) {
            hipLaunchKernelGGL((flash_fwd_kernel<64, PF_ROWS, 1, 8, false>), g, block, 0, st, b);
            return hipGetLastError();
        }
#define F(HD, KIND, NQ)                                                                    \
    if (hd == HD && kind == KIND && nqt == NQ) {                                           \
        hipLaunchKernelGGL((flash_fwd_kernel<HD, KIND, NQ, PW, false>), g, block, 0, st, b); \
        return hipGetLastError();                                                          \
    }
#define FQ(HD, KIND, NQ)                                                                   \
    if (hd == HD && kind == KIND && nqt == NQ && ql) {                                     \
        hipLaunchKernelGGL((flash_fwd_kernel<HD, KIND, NQ, PW, true>), g, block, 0, st, b); \
        return hipGetLastError();                                                          \
    }
        FQ(64, PF_F16, 1) FQ(128, PF_F16, 1) FQ(64, PF_T16, 1) FQ(128, PF_T16, 1)
        F(64, PF_F16, 1) F(64, PF_F16, 2) F(128, PF_F16, 1) F(128, PF_F16, 2)
        F(64, PF_T16, 1) F(64, PF_T16, 2) F(128, PF_T16, 1) F(128, PF_T16, 2)
        F(64, PF_F32, 1) F(64, PF_F32, 2) F(128, PF_F32, 1) F(128, PF_F32, 2)
        F(64, PF_ROWS, 1) F(64, PF_ROWS, 2)
#undef FQ
#undef F
    }
    LK(64, PF_F16) LK(128, PF_F16) LK(64, PF_F32) LK(128, PF_F32) LK(64, PF_ROWS) LK(64, PF_T16) LK(128, PF_T16)
#undef LK
#undef L
    return hipErrorInvalidValue;
}

}  // namespace llmtie
