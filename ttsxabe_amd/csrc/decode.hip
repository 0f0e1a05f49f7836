// Split-K single-token decode attention for gfx950.
//
// Replaces the reference's `attn_decode_impl` / `attn_decode_run_impl` /
// `ad_publish_merge` (crates/llmtie-cuda/src/kernels.rs:5779-6505) with one
// MFMA kernel, templated on the head width and on the cache's storage:
//   KV_F16 - K [kv][cap][hd] f16, V [kv][hd][cap] f16 (the reference layout)
//   KV_F32 - the same layout at f32 (the Whisper decoder's self cache)
//   KV_T16 - the tiled f16 layout of kvlayout.h (fragment order)
//   KV_TQ8 - the tiled GGUF Q8_0 layout of kvlayout.h (32 int8 codes + one f16
//            scale per 32 dims of a position), for batched sequences in slots.
// The tiled layouts make every K/V load a contiguous 1 KB wave-wide read; off
// the reference layout a load instruction touches 16 rows, which measured at
// about half the achievable HBM rate for the same bytes.
//
// Work decomposition. A workgroup is four waves on one (sequence, kv head,
// split); a split is `4 * nit` blocks of 32 consecutive keys and wave w takes
// blocks w, w + 4, ... of it. All the query heads of the GQA group (<= 16)
// ride in the 16 columns of one MFMA tile, so every K/V byte is read once per
// group, as the reference's shared-group design does.
//
// Per 32-key block a wave computes S^T = K Q^T (A = 16 keys x 32 dims from
// HBM, B = queries in registers) for two 16-key tiles. Tile T's A-row m is key
// 8*(m/4) + 4T + m%4, which makes D-row 4*grp + r of tile T key
// 8*grp + 4T + r: after both tiles lane l holds the scores of keys
// 8*grp + 0..7 for query `col`, exactly the B-operand slots of the value
// product O^T = V^T P^T over those 32 keys. The probabilities therefore never
// leave registers, and the V^T operand is one 16-byte run of a value row.
//
// Arithmetic. The reference's decode is an f32 computation (f32 query times
// f16 or f32 cache, f32 probabilities). To stay within its tolerance the f32
// operands go into the MFMA as hi + lo f16 pairs (query, probabilities, and
// f32 cache values), which carries ~22 bits; f16 and int8 cache values are
// exact in f16. The softmax runs in log2 units with v_exp_f32.
//
// Merge. Each wave keeps a running (m, l, O); the four waves combine through
// LDS in a fixed order; a multi-split head publishes (m, l, O) to scratch and
// the last workgroup of the head (agent-scope counter) merges all splits in
// split order and resets the counter to zero. The result does not depend on
// which workgroup finishes last, so repeated calls are bit-identical.
#include <type_traits>
#include "common.h"
#include "decode.h"
#include "kvlayout.h"

namespace llmtie {

constexpr int DW = 4;                 // waves per workgroup
constexpr int DT = DW * LLMTIE_WAVE;  // threads per workgroup

// Eight offset-binary codes u = code + 128 (two dwords) as the halves
// 1152 + code: each byte spliced under the exponent byte 0x64 is the half
// 1024 + u. Exact, and two instructions per pair.
__device__ __forceinline__ half8 dq8_biased(uint32_t w0, uint32_t w1) {
    const uint32_t p[4] = {__builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u)};
    half8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r[2 * i] = __builtin_bit_cast(half_t, (uint16_t)(p[i] & 0xffffu));
        r[2 * i + 1] = __builtin_bit_cast(half_t, (uint16_t)(p[i] >> 16));
    }
    return r;
}
// The same with the 1152 taken off (one packed f16 add per pair): the codes.
__device__ __forceinline__ half8 dq8(uint32_t w0, uint32_t w1) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const half8 b = dq8_biased(w0, w1);
    const h2 bias = {(half_t)1152.0f, (half_t)1152.0f};
    half8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const h2 v = h2{b[2 * i], b[2 * i + 1]} - bias;
        r[2 * i] = v[0];
        r[2 * i + 1] = v[1];
    }
    return r;
}

template <int HD, int KIND>
struct Frag;

template <int HD>
struct Frag<HD, KV_F16> {
    half8 k[2][HD / 32];
    half8 v[HD / 16];
};
template <int HD>
struct Frag<HD, KV_T16> {
    half8 k[2][HD / 32];
    half8 v[HD / 16];
};
template <int HD>
struct Frag<HD, KV_F32> {
    half8 kh[2][HD / 32], kl[2][HD / 32];
    half8 vh[HD / 16], vl[HD / 16];
};
// Raw codes and scales, dequantised where they are used.
template <int HD>
struct Frag<HD, KV_TQ8> {
    uint4 kc[2][HD / 64];  // (T, step pair)
    uint4 vc[HD / 32];     // tile pair
    uint4 ks[HD / 32];     // per dim block: the scales of keys 8g .. 8g+7
    uint4 vs[HD / 32];
};

struct Ctx {
    const char* k;   // reference layouts: K base of this kv head; tiled: block 0 of this (slot, kv head)
    const char* v;   // reference layouts: V^T base of this kv head
    long bstride;    // tiled: bytes per block
    int tk, cap;
};

// Keys key0 .. key0 + 7 of one V^T row (rb: the row's first element) of the
// reference layout, as f16 hi/lo or exact f16. VA is the alignment the row
// start guarantees (16 or 8 bytes), which makes the row a whole number of
// granules (VA bytes); a granule that would pass the cache's capacity is read
// from the row's start instead (its keys are past tk, and the fold zeroes
// them), so no block reads outside the row, whatever tk.
template <int KIND, int VA, bool NTL = false>
__device__ __forceinline__ void v_row8(const Ctx& c, size_t rb, int key0, half8& h, half8& l) {
    constexpr int ESZ = KIND == KV_F16 ? 2 : 4, G = VA / ESZ;  // elements per granule
    auto at = [&](int g) { return rb + (key0 + G * (g + 1) <= c.cap ? key0 + G * g : 0); };
    if constexpr (KIND == KV_F16) {
        const uint16_t* v = reinterpret_cast<const uint16_t*>(c.v);
        if constexpr (VA == 16) {
            h = NTL ? __builtin_nontemporal_load(reinterpret_cast<const half8*>(v + at(0))) : ld_h8(v + at(0));
        } else {
            const uint2 a = *reinterpret_cast<const uint2*>(v + at(0));
            const uint2 b = *reinterpret_cast<const uint2*>(v + at(1));
            const uint32_t w[4] = {a.x, a.y, b.x, b.y};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h[2 * i] = __builtin_bit_cast(half_t, (uint16_t)(w[i] & 0xffffu));
                h[2 * i + 1] = __builtin_bit_cast(half_t, (uint16_t)(w[i] >> 16));
            }
        }
    } else {
        const float* v = reinterpret_cast<const float*>(c.v);
        float x[8];
        if constexpr (VA == 16) {
            const float4 a = *reinterpret_cast<const float4*>(v + at(0));
            const float4 b = *reinterpret_cast<const float4*>(v + at(1));
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
            x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
        } else {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float2 a = *reinterpret_cast<const float2*>(v + at(g));
                x[2 * g] = a.x;
                x[2 * g + 1] = a.y;
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            half_t hh, ll;
            split_h(x[j], hh, ll);
            h[j] = hh;
            l[j] = ll;
        }
    }
}

// 16 bytes of a stream read once, with the non-temporal hint.
__device__ __forceinline__ uint4 ld_stream16(const uint4* p) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const v4u x = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(x[0], x[1], x[2], x[3]);
}

// Loads the 32-key block starting at p0 (block index p0 / 32).
// Tiled layouts: straight 16-byte-per-lane reads, always in bounds (a tiled
// cache holds whole blocks); keys >= tk are dropped later by the fold. Each
// instruction reads whole 1 KB runs that nothing reads again in the launch,
// so they are non-temporal (C2 9.86 -> 9.43 us). The reference layouts'
// 16-byte pieces are non-temporal (NTL) on the MFMA path (C2 reference
// layout 10.16 -> 9.94 us) but not on the group-1 path, whose loads share
// lines in a pattern the evict-first policy hurts (the MHA decode at 4000
// positions went 22.1 -> 23.9 us).
// Reference layouts: every block is read the same way, the context's partial
// last block included: K rows past the capacity are clamped to its last row,
// V granules past it to the row's start (v_row8), so nothing outside the
// cache is read, and whatever lies past tk is left to the fold's mask (scores
// to -inf, values to zero).
template <int HD, int KIND, int VA, bool NTL = false>
__device__ __forceinline__ void load_block(const Ctx& c, int p0, int lane, Frag<HD, KIND>& f) {
    constexpr int NS = HD / 32;
    constexpr int NT = HD / 16;
    const int col = lane & 15, grp = lane >> 4;
    if constexpr (KIND == KV_T16) {
        const half8* b = reinterpret_cast<const half8*>(c.k + (long)(p0 >> 5) * c.bstride);
        // In the order the fold consumes them (dim block s outer, key tile T inner).
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int T = 0; T < 2; ++T) f.k[T][s] = __builtin_nontemporal_load(&b[(T * NS + s) * 64 + lane]);
        const half8* vb = b + 4 * HD;  // the V area: 32*HD halves in
#pragma unroll
        for (int t = 0; t < NT; ++t) f.v[t] = __builtin_nontemporal_load(&vb[t * 64 + lane]);
    } else if constexpr (KIND == KV_TQ8) {
        const char* b = c.k + (long)(p0 >> 5) * c.bstride;
        const uint4* kc = reinterpret_cast<const uint4*>(b);
        const uint4* vc = reinterpret_cast<const uint4*>(b + 32 * HD);
        const uint4* ks = reinterpret_cast<const uint4*>(b + 64 * HD);
        const uint4* vs = reinterpret_cast<const uint4*>(b + 64 * HD + 64 * (HD / 32));
#pragma unroll
        for (int T = 0; T < 2; ++T)
#pragma unroll
            for (int sp = 0; sp < NS / 2; ++sp) f.kc[T][sp] = ld_stream16(&kc[(T * (NS / 2) + sp) * 64 + lane]);
#pragma unroll
        for (int tp = 0; tp < NT / 2; ++tp) f.vc[tp] = ld_stream16(&vc[tp * 64 + lane]);
        // Dim block i, keys 8*grp .. +7: one 16-byte piece per block.
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            f.ks[i] = ks[i * 4 + grp];
            f.vs[i] = vs[i * 4 + grp];
        }
    } else {
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            const int kk = min(p0 + 8 * (col >> 2) + 4 * T + (col & 3), c.cap - 1);
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const int d0 = 32 * s + 8 * grp;
                if constexpr (KIND == KV_F16) {
                    const half8* kp = reinterpret_cast<const half8*>(c.k + ((size_t)kk * HD + d0) * 2);
                    f.k[T][s] = NTL ? __builtin_nontemporal_load(kp) : *kp;
                } else {
                    const float4* p = reinterpret_cast<const float4*>(c.k + ((size_t)kk * HD + d0) * 4);
                    const float4 a = p[0], b = p[1];
                    const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                    half8 h, l;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        half_t hh, ll;
                        split_h(x[j], hh, ll);
                        h[j] = hh;
                        l[j] = ll;
                    }
                    f.kh[T][s] = h;
                    f.kl[T][s] = l;
                }
            }
        }
        const int kb = p0 + 8 * grp;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            half8 h = zero_h8(), l = zero_h8();
            v_row8<KIND, VA, NTL>(c, (size_t)(16 * t + col) * c.cap, kb, h, l);
            if constexpr (KIND == KV_F32) {
                f.vh[t] = h;
                f.vl[t] = l;
            } else {
                f.v[t] = h;
            }
        }
    }
}

// Half j of a 16-byte piece (keys 8g+j .. for scales: element e).
__device__ __forceinline__ half_t h_at(const uint4& u, int e) {
    const uint32_t w = e < 2 ? u.x : e < 4 ? u.y : e < 6 ? u.z : u.w;
    return __builtin_bit_cast(half_t, (uint16_t)((e & 1) ? (w >> 16) : (w & 0xffffu)));
}

// One 32-key block folded into the wave's running softmax state. MASK: keys
// >= tk are dropped (only the partial block needs it).
template <int HD, int KIND, bool MASK>
__device__ __forceinline__ void fold_block(const Frag<HD, KIND>& f, const half8 (&qh)[HD / 32],
                                           const half8 (&ql)[HD / 32],
                                           int p0, int tk, int grp,
                                           float score_l2, float& m_run, float& l_run,
                                           floatx4 (&o)[HD / 16]) {
    constexpr int NS = HD / 32;
    constexpr int NT = HD / 16;
    float sc[8];
    // The two key tiles' chains interleaved (s outer, T inner): each tile's
    // accumulation order is unchanged, and the matrix unit always has an
    // independent product to start while the other tile's waits on its
    // predecessor.
    floatx4 accs[2] = {zero_f4(), zero_f4()};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            floatx4& acc = accs[T];
            if constexpr (KIND == KV_F16 || KIND == KV_T16) {
                acc = mfma16(f.k[T][s], qh[s], acc);
                acc = mfma16(f.k[T][s], ql[s], acc);
            } else if constexpr (KIND == KV_F32) {
                acc = mfma16(f.kh[T][s], qh[s], acc);
                acc = mfma16(f.kh[T][s], ql[s], acc);
                acc = mfma16(f.kl[T][s], qh[s], acc);
            } else {
                // K enters as exact f16 codes (the 1152 offset taken off
                // before the product: left in, it would cancel against the f32
                // accumulator and cost ~1e-3 of score precision), scaled per
                // dim block after the product.
                const uint4& w = f.kc[T][s >> 1];
                const half8 kq = (s & 1) ? dq8(w.z, w.w) : dq8(w.x, w.y);
                floatx4 b = mfma16(kq, qh[s], zero_f4());
                b = mfma16(kq, ql[s], b);
                // Key 8g + 4T + r, dim block s: half 4T + r of the block's scale piece.
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] += (float)h_at(f.ks[s], 4 * T + r) * b[r];
            }
        }
    }
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[4 * T + r] = accs[T][r];
    const int kb = p0 + 8 * grp;
    float mx = ninf();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sc[j] = (!MASK || kb + j < tk) ? sc[j] : ninf();
        mx = fmaxf(mx, sc[j]);
    }
    mx = max4grp(mx);
    const float mn = fmaxf(m_run, mx);
    const float fac = ex2(m_run - mn);
    m_run = mn;
    // Q8_0: probabilities carry a factor 2^10 (in l and O alike, so O / l is
    // unchanged), which keeps P' = P * d_v (d_v ~ 1e-2) clear of the f16
    // subnormal range where its relative precision would fall away.
    const float mb = KIND == KV_TQ8 ? mn - 10.0f : mn;
    float p[8], ps = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        p[j] = ex2(sc[j] - mb);
        ps += p[j];
    }
    l_run = l_run * fac + ps;
    // Once the running max has settled it rarely moves: skip the rescale of
    // the context when no lane's factor differs from one.
    if (__any(fac != 1.0f)) {
#pragma unroll
        for (int t = 0; t < NT; ++t) o[t] *= fac;
    }

    if constexpr (KIND == KV_TQ8) {
        // P' = P * d_v (the scale of each key's dim block) as one f16 operand
        // per dim block, formed with packed f16 multiplies: Q8_0 values carry
        // 8 bits, so the 11 of an f16 P' keep the product well inside the
        // quantisation's own error.
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        h2 ph[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a0 = (!MASK || kb + 2 * i < tk) ? p[2 * i] : 0.0f;
            const float a1 = (!MASK || kb + 2 * i + 1 < tk) ? p[2 * i + 1] : 0.0f;
            ph[i] = h2{to_h(a0), to_h(a1)};
        }
#pragma unroll
        for (int b = 0; b < NS; ++b) {
            const uint32_t dw[4] = {f.vs[b].x, f.vs[b].y, f.vs[b].z, f.vs[b].w};
            half8 pv;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h2 d = __builtin_bit_cast(h2, dw[i]);
                if constexpr (MASK) {
                    // a tail key's scale may be any bit pattern: zero it too
                    if (kb + 2 * i >= tk) d[0] = (half_t)0.0f;
                    if (kb + 2 * i + 1 >= tk) d[1] = (half_t)0.0f;
                }
                const h2 x = ph[i] * d;
                pv[2 * i] = x[0];
                pv[2 * i + 1] = x[1];
            }
#pragma unroll
            for (int t = 2 * b; t < 2 * b + 2; ++t) {
                const uint4& w = f.vc[t >> 1];
                const half8 vq = (t & 1) ? dq8(w.z, w.w) : dq8(w.x, w.y);
                o[t] = mfma16(vq, pv, o[t]);
            }
        }
    } else {
        half8 ph, pl;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            half_t hh, ll;
            split_h(p[j], hh, ll);
            ph[j] = hh;
            pl[j] = ll;
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if constexpr (KIND == KV_F16 || KIND == KV_T16) {
                // A cache may hold anything past tk (the tiled cache's block
                // tail, the reference layout's unused capacity, clamped reads):
                // zero those keys' values so that 0 * (a non-finite half)
                // cannot reach the sum.
                half8 vv = f.v[t];
                if constexpr (MASK) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) vv[j] = (kb + j < tk) ? vv[j] : (half_t)0.0f;
                }
                o[t] = mfma16(vv, ph, o[t]);
                o[t] = mfma16(vv, pl, o[t]);
            } else {
                half8 vh = f.vh[t], vl = f.vl[t];
                if constexpr (MASK) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        vh[j] = (kb + j < tk) ? vh[j] : (half_t)0.0f;
                        vl[j] = (kb + j < tk) ? vl[j] : (half_t)0.0f;
                    }
                }
                o[t] = mfma16(vh, ph, o[t]);
                o[t] = mfma16(vh, pl, o[t]);
                o[t] = mfma16(vl, ph, o[t]);
            }
        }
    }
}

// One tiled Q8_0 block folded into the wave's running softmax state: the
// arithmetic of fold_block<HD, KV_TQ8>, bit for bit, in an order that keeps
// the matrix unit and the VALU busy together (one wave per SIMD issues a
// VALU instruction only every ~6-7 clocks, so the stream-K kernel's blocks
// cost their VALU count). Every K fragment is dequantised first; the sixteen
// score MFMAs (hi halves of the queries, then lo, so no MFMA waits on the one
// before it) run while the V fragments are dequantised; the scaled scores,
// the softmax and P' follow, and the value MFMAs close the block.
// (Codes entering the MFMAs biased, 1152 + code, with the bias cancelled in
// the accumulator: for V no loss and no gain; for K the score accumulators
// lost precision to 1.07e-3 of full scale on 8-key sequences, not kept.)
template <int HD, bool MASK>
__device__ __forceinline__ void fold_block_q8(const Frag<HD, KV_TQ8>& f, const half8 (&qh)[HD / 32],
                                              const half8 (&ql)[HD / 32], int p0, int tk, int grp,
                                              float& m_run, float& l_run, floatx4 (&o)[HD / 16]) {
    constexpr int NS = HD / 32;
    constexpr int NT = HD / 16;
    half8 kq[2][NS];
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const uint4& w = f.kc[T][s >> 1];
            kq[T][s] = (s & 1) ? dq8(w.z, w.w) : dq8(w.x, w.y);
        }
    floatx4 b[2][NS];
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int s = 0; s < NS; ++s) b[T][s] = mfma16(kq[T][s], qh[s], zero_f4());
    half8 vq[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const uint4& w = f.vc[t >> 1];
        vq[t] = (t & 1) ? dq8(w.z, w.w) : dq8(w.x, w.y);
    }
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int s = 0; s < NS; ++s) b[T][s] = mfma16(kq[T][s], ql[s], b[T][s]);
    float sc[8];
#pragma unroll
    for (int T = 0; T < 2; ++T) {
        floatx4 acc = zero_f4();
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] += (float)h_at(f.ks[s], 4 * T + r) * b[T][s][r];
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[4 * T + r] = acc[r];
    }
    const int kb = p0 + 8 * grp;
    float mx = ninf();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sc[j] = (!MASK || kb + j < tk) ? sc[j] : ninf();
        mx = fmaxf(mx, sc[j]);
    }
    mx = max4grp(mx);
    const float mn = fmaxf(m_run, mx);
    const float fac = ex2(m_run - mn);
    m_run = mn;
    // Probabilities carry a factor 2^10 (see fold_block).
    const float mb = mn - 10.0f;
    float p[8], ps = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        p[j] = ex2(sc[j] - mb);
        ps += p[j];
    }
    l_run = l_run * fac + ps;
    if (__any(fac != 1.0f)) {
#pragma unroll
        for (int t = 0; t < NT; ++t) o[t] *= fac;
    }
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 ph[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a0 = (!MASK || kb + 2 * i < tk) ? p[2 * i] : 0.0f;
        const float a1 = (!MASK || kb + 2 * i + 1 < tk) ? p[2 * i + 1] : 0.0f;
        ph[i] = h2{to_h(a0), to_h(a1)};
    }
#pragma unroll
    for (int bb = 0; bb < NS; ++bb) {
        const uint32_t dw[4] = {f.vs[bb].x, f.vs[bb].y, f.vs[bb].z, f.vs[bb].w};
        half8 pv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h2 d = __builtin_bit_cast(h2, dw[i]);
            if constexpr (MASK) {
                if (kb + 2 * i >= tk) d[0] = (half_t)0.0f;
                if (kb + 2 * i + 1 >= tk) d[1] = (half_t)0.0f;
            }
            const h2 x = ph[i] * d;
            pv[2 * i] = x[0];
            pv[2 * i + 1] = x[1];
        }
#pragma unroll
        for (int t = 2 * bb; t < 2 * bb + 2; ++t) o[t] = mfma16(vq[t], pv, o[t]);
    }
}

// One element of the context, and its int8 twin: the 32 threads of a scale
// group are 32 consecutive lanes of one wave (the caller guarantees it).
__device__ __forceinline__ void emit(float* out, int8_t* tc, float* ts, size_t idx, float y) {
    out[idx] = y;
    if (tc) {
        float mx = fabsf(y);
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        const float d = mx * (1.0f / 127.0f);
        const float inv = d > 0.0f ? 1.0f / d : 0.0f;
        tc[idx] = (int8_t)(int)rintf(y * inv);
        if ((threadIdx.x & 31) == 0) ts[idx >> 5] = d;
    }
}

// The merge of one head's split partials, in split order, by one workgroup
// of DT threads, with every load issued before any is waited on (one memory
// round trip): first the (m, l) pairs the weights need, then the partial
// columns, so the weights are computed while the columns are in flight.
// AUX: the cache policy of the partial loads (ld_region4): AUX_AGENT for
// partials handed over with coherent stores inside this launch, AUX_XCD for
// partials stored into this XCD's L2 inside this launch, 0 when a launch
// boundary separates writer and reader. `lds` holds >= 4096 floats.
// Thread t owns float4 column c = t % C of the [g][HD] partial (C = n / 4)
// and the splits s = t / C, t / C + R, ... (R = DT / C phases).
template <int HD, int AUX>
__device__ __forceinline__ void merge_head(const float* po, const float* pml, int nsplit, int group, float* lds,
                                           float* gl, float* out, int8_t* tc, float* ts, size_t obase) {
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int n = group * HD;
    const int C = n / 4;
    const int R = C >= DT ? 1 : DT / C;
    float* red = lds;          // [R][n] per-phase sums (<= 2048 floats)
    float* wts = lds + 2048;   // [nsplit][group] weights (<= 1024 floats)
    const Region ro = region(po, (uint32_t)((size_t)nsplit * n * 4));
    const Region rml = region(pml, (uint32_t)((size_t)nsplit * group * 8));

    // (m, l) of query head g0 = wave for splits lane + 64k. Every load here
    // is unconditional (past the regions' ends the buffer bounds check
    // returns zeros), so the compiler can count them and the weights wait
    // only for the (m, l) loads, not for the partial columns behind them.
    constexpr int MK = DECODE_MAX_SPLITS / 64;
    constexpr uint32_t OUT = 0x80000000u;  // an offset past any region (all are < 2 GB)
    float2 ml[MK];
    const int g0 = wave;
#pragma unroll
    for (int k = 0; k < MK; ++k)
        ml[k] = ld_region2<AUX>(rml, 64 * k < nsplit && g0 < group ? (uint32_t)(((lane + 64 * k) * group + g0) * 8) : OUT);
    __builtin_amdgcn_sched_barrier(0);  // the (m, l) loads go out first
    // This thread's partial columns, up to U splits in flight.
    constexpr int U = 16;
    const int c4 = tid % C, phase = tid / C;
    const bool has = tid < R * C;
    float4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int sp = phase + u * R;
        x[u] = ld_region4<AUX>(ro, has && sp < nsplit ? (uint32_t)(((size_t)sp * n + 4 * c4) * 4) : OUT);
    }
    // Weights: for query head g (a wave per g), M_g = max_s m, w_sg = 2^(m - M),
    // L_g = sum_s l w, reduced across the wave's lanes.
    for (int g = wave; g < group; g += DW) {
        if (g != g0) {
#pragma unroll
            for (int k = 0; k < MK; ++k)
                if (64 * k < nsplit) ml[k] = ld_region2<AUX>(rml, (uint32_t)(((lane + 64 * k) * group + g) * 8));
        }
        float mx = ninf();
#pragma unroll
        for (int k = 0; k < MK; ++k)
            if (lane + 64 * k < nsplit) mx = fmaxf(mx, ml[k].x);
        mx = wave_max(mx);
        float L = 0.0f;
#pragma unroll
        for (int k = 0; k < MK; ++k) {
            const int sp = lane + 64 * k;
            if (sp < nsplit) {
                const float w = ex2(ml[k].x - mx);
                wts[sp * group + g] = w;
                L += ml[k].y * w;
            }
        }
        L = wave_sum(L);
        if (lane == 0) gl[g] = L;
    }
    __syncthreads();
    if (has) {
        const int g = (4 * c4) / HD;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int sp = phase + u * R;
            const float wt = sp < nsplit ? wts[sp * group + g] : 0.0f;
            acc.x += x[u].x * wt;
            acc.y += x[u].y * wt;
            acc.z += x[u].z * wt;
            acc.w += x[u].w * wt;
        }
        // Splits beyond the first U * R (long contexts): more rounds.
        for (int s0 = phase + U * R; s0 < nsplit; s0 += U * R) {
#pragma unroll
            for (int u = 0; u < U; ++u) x[u] = ld_region4<AUX>(ro, (uint32_t)(((size_t)(s0 + u * R) * n + 4 * c4) * 4));
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int sp = s0 + u * R;
                const float wt = sp < nsplit ? wts[sp * group + g] : 0.0f;
                acc.x += x[u].x * wt;
                acc.y += x[u].y * wt;
                acc.z += x[u].z * wt;
                acc.w += x[u].w * wt;
            }
        }
        reinterpret_cast<float4*>(red + phase * n)[c4] = acc;
    }
    // Columns beyond DT (C > DT): the remaining work items, one round each.
    for (int w = tid + DT; w < C; w += DT) {
        const int g = (4 * w) / HD;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int sp = 0; sp < nsplit; ++sp) {
            const float4 y = ld_region4<AUX>(ro, (uint32_t)(((size_t)sp * n + 4 * w) * 4));
            const float wt = wts[sp * group + g];
            acc.x += y.x * wt;
            acc.y += y.y * wt;
            acc.z += y.z * wt;
            acc.w += y.w * wt;
        }
        reinterpret_cast<float4*>(red)[w] = acc;
    }
    __syncthreads();
    // Sum the phases. R (1 to 16) is fixed by the head's shape; with a
    // compile-time bound every LDS read of an element is issued before the
    // first is waited on (a runtime-bounded sum waited on each read in turn).
    // Reads are clamped to the R rows written and the sum masked to them.
    auto finish = [&](auto rr) {
        constexpr int RR = decltype(rr)::value;
        for (int e = tid; e < n; e += DT) {
            float v[RR];
#pragma unroll
            for (int r = 0; r < RR; ++r) v[r] = red[min(r, R - 1) * n + e];
            float acc = 0.0f;
#pragma unroll
            for (int r = 0; r < RR; ++r) acc += r < R ? v[r] : 0.0f;
            emit(out, tc, ts, obase + e, acc / gl[e / HD]);
        }
    };
    switch (R) {
        case 1: finish(std::integral_constant<int, 1>{}); break;
        case 2: finish(std::integral_constant<int, 2>{}); break;
        case 4: finish(std::integral_constant<int, 4>{}); break;
        case 8: finish(std::integral_constant<int, 8>{}); break;
        default: finish(std::integral_constant<int, 16>{}); break;  // any other R <= 16
    }
}


// ------------------------------------------------------------------------
// Group-1 (MHA) decode on the VALU. With one query head per kv head an MFMA
// tile would carry one live column of 16, and an f32 operand would need hi +
// lo f16 halves; here every product is an f32 FMA (f16 cache values convert
// exactly), as in the reference's own f32 arithmetic.
//
// The block's K and V arrive in the same fragment order as for the MFMA path
// (lane (col, grp) holds key 8*(col/4) + 4T + col%4, dims 32s + 8grp .. +7 of
// K, and dim 16t + col, keys 8grp .. +7 of V): a lane's partial dot products
// over its 8 * HD/32 dims are summed over the four lanes of its column
// (sum4grp), the block's probabilities go through a 32-float LDS row so each
// lane can read the eight it needs for V, and a lane's context sums for dims
// 16t + col are summed over the four grp lanes once, after the last block.

// f32 cache values for the VALU fold (no hi/lo split).
template <int HD>
struct FragF32 {
    float4 k[2][HD / 32][2];
    float4 v[HD / 16][2];
};

// The 32-key block at p0 of an f32 reference-layout cache, raw, read as
// load_block reads it (rows and granules clamped inside the capacity).
template <int HD, int VA>
__device__ __forceinline__ void load_block_f32v(const Ctx& c, int p0, int lane, FragF32<HD>& f) {
    constexpr int NS = HD / 32, NT = HD / 16;
    const int col = lane & 15, grp = lane >> 4;
    const float* kb = reinterpret_cast<const float*>(c.k);
    const float* vb = reinterpret_cast<const float*>(c.v);
#pragma unroll
    for (int T = 0; T < 2; ++T) {
        const int kk = min(p0 + 8 * (col >> 2) + 4 * T + (col & 3), c.cap - 1);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const float4* p = reinterpret_cast<const float4*>(kb + (size_t)kk * HD + 32 * s + 8 * grp);
            f.k[T][s][0] = p[0];
            f.k[T][s][1] = p[1];
        }
    }
    const int k0 = p0 + 8 * grp;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const size_t rb = (size_t)(16 * t + col) * c.cap;
        auto at = [&](int g, int G) { return vb + rb + (k0 + G * (g + 1) <= c.cap ? k0 + G * g : 0); };
        if constexpr (VA == 16) {
            f.v[t][0] = *reinterpret_cast<const float4*>(at(0, 4));
            f.v[t][1] = *reinterpret_cast<const float4*>(at(1, 4));
        } else {
            const float2 a0 = *reinterpret_cast<const float2*>(at(0, 2)), a1 = *reinterpret_cast<const float2*>(at(1, 2));
            const float2 a2 = *reinterpret_cast<const float2*>(at(2, 2)), a3 = *reinterpret_cast<const float2*>(at(3, 2));
            f.v[t][0] = make_float4(a0.x, a0.y, a1.x, a1.y);
            f.v[t][1] = make_float4(a2.x, a2.y, a3.x, a3.y);
        }
    }
}

// The f32 cache at head_dim 64 in line order. The fragment order above has
// each load instruction touch 16 keys (or 16 V rows) in sixteen 128-byte
// lines, half of each; a workgroup of a launch that occupies few CUs is then
// bound by its CU's line rate, not by HBM. Here every instruction reads eight
// whole lines (1 KB), and the fold is arranged around that:
//   K: instruction i holds keys 4i + lane/16, dims 4 (lane%16) .. +3, so a
//      lane's query slice is 4 dims and a key's dot product is spread over
//      the 16 lanes of a DPP row;
//   V: instruction i holds rows (dims) 8i + lane/8, keys 4 (lane%8) .. +3.
template <int HD>
struct FragF32L {
    static_assert(HD == 64, "line-order f32 fold: head_dim 64");
    float4 k[8];
    float4 v[8];
};

template <int HD, int VA>
__device__ __forceinline__ void load_block_f32l(const Ctx& c, int p0, int lane, FragF32L<HD>& f) {
    const float* kb = reinterpret_cast<const float*>(c.k);
    const float* vb = reinterpret_cast<const float*>(c.v);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int key = min(p0 + 4 * i + (lane >> 4), c.cap - 1);
        f.k[i] = *reinterpret_cast<const float4*>(kb + (size_t)key * HD + 4 * (lane & 15));
    }
    const int k0 = p0 + 4 * (lane & 7);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // Granules past the capacity read from the row's start (see v_row8).
        const float* rb = vb + (size_t)(8 * i + (lane >> 3)) * c.cap;
        if constexpr (VA == 16) {
            f.v[i] = *reinterpret_cast<const float4*>(rb + (k0 + 4 <= c.cap ? k0 : 0));
        } else {
            const float2 a0 = *reinterpret_cast<const float2*>(rb + (k0 + 2 <= c.cap ? k0 : 0));
            const float2 a1 = *reinterpret_cast<const float2*>(rb + (k0 + 4 <= c.cap ? k0 + 2 : 0));
            f.v[i] = make_float4(a0.x, a0.y, a1.x, a1.y);
        }
    }
}

// One step of a reduce-scatter across a lane pair that differs in bit B of
// the lane id (DPP control CTRL selects the partner): of the 2n values, the
// lane keeps the upper n when its bit B is set, the lower n otherwise, and
// adds the partner's copies of the same n. Partners keep opposite halves.
template <int CTRL, int B, int N>
__device__ __forceinline__ void rs_step(const float (&x)[2 * N], float (&y)[N], int lane) {
    const bool up = (lane >> B) & 1;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const float keep = up ? x[N + k] : x[k];
        const float send = up ? x[k] : x[N + k];
        y[k] = keep + dpp_f<CTRL>(send);
    }
}

// One 32-key block of the line-order f32 cache folded into the wave's
// running (m, l, o). qv: the lane's query dims 4 (lane%16) .. +3 in log2-score
// units; o[i]: the lane's context sum for dim 8i + lane/8 over keys
// 4 (lane%8) .. +3 of every block; pw: the wave's 32-float LDS row.
template <int HD, bool MASK>
__device__ __forceinline__ void fold_block_g1l(const FragF32L<HD>& f, const float (&qv)[4], int p0, int tk,
                                               int lane, float& m_run, float& l_run, float (&o)[8], float* pw) {
    float d[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float acc = f.k[i].x * qv[0];
        acc = __builtin_fmaf(f.k[i].y, qv[1], acc);
        acc = __builtin_fmaf(f.k[i].z, qv[2], acc);
        d[i] = __builtin_fmaf(f.k[i].w, qv[3], acc);
    }
    // Sum each key's 16 partial dots over its DPP row: row mirror (bit 3),
    // half-row mirror (bit 2), quad xor 3 (bit 1) scatter the eight keys,
    // quad xor 1 completes the pair. Lane ends with key 4 ((lane/2)%8) + lane/16,
    // as does its xor-1 partner.
    float d4[4], d2[2], d1[1];
    rs_step<0x140, 3, 4>(d, d4, lane);
    rs_step<0x141, 2, 2>(d4, d2, lane);
    rs_step<0x1b, 1, 1>(d2, d1, lane);
    float sc = d1[0] + dpp_f<0xb1>(d1[0]);
    const int kl = 4 * ((lane >> 1) & 7) + (lane >> 4);
    if constexpr (MASK) sc = p0 + kl < tk ? sc : ninf();
    const float mn = fmaxf(m_run, wave_max(sc));
    const float fac = ex2(m_run - mn);
    m_run = mn;
    const float e = ex2(sc - mn);
    // Each key's probability sits in two lanes: half the wave sum is the
    // block's (an exact scaling).
    l_run = l_run * fac + wave_sum(e) * 0.5f;
    if (__any(fac != 1.0f)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] *= fac;
    }
    if (!(lane & 1)) pw[kl] = e;
    __builtin_amdgcn_wave_barrier();
    const float4 pp = *reinterpret_cast<const float4*>(pw + 4 * (lane & 7));
    const int k0 = p0 + 4 * (lane & 7);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float4 v = f.v[i];
        if constexpr (MASK) {
            // Values past tk may be anything (unused capacity, clamped reads).
            v.x = k0 < tk ? v.x : 0.0f;
            v.y = k0 + 1 < tk ? v.y : 0.0f;
            v.z = k0 + 2 < tk ? v.z : 0.0f;
            v.w = k0 + 3 < tk ? v.w : 0.0f;
        }
        float acc = __builtin_fmaf(pp.x, v.x, o[i]);
        acc = __builtin_fmaf(pp.y, v.y, acc);
        acc = __builtin_fmaf(pp.z, v.z, acc);
        o[i] = __builtin_fmaf(pp.w, v.w, acc);
    }
    __builtin_amdgcn_wave_barrier();  // the row is read before the next block's writes
}

// The line-order context sums reduced over the eight lanes that share a dim
// row: lane ends with dim 8 (lane%8) + lane/8 (half-row mirror, quad xor 3,
// quad xor 1 scatter the eight dims).
__device__ __forceinline__ float g1l_context(const float (&o)[8], int lane) {
    float o4[4], o2[2], o1[1];
    rs_step<0x141, 2, 4>(o, o4, lane);
    rs_step<0x1b, 1, 2>(o4, o2, lane);
    rs_step<0xb1, 0, 1>(o2, o1, lane);
    return o1[0];
}

// Element j of a lane's 8-element K or V run, as f32.
template <int HD, int KIND, typename FR>
__device__ __forceinline__ float g1_k(const FR& f, int T, int s, int j) {
    if constexpr (KIND == KV_F32) {
        const float4& x = f.k[T][s][j >> 2];
        return (j & 3) == 0 ? x.x : (j & 3) == 1 ? x.y : (j & 3) == 2 ? x.z : x.w;
    } else {
        return (float)f.k[T][s][j];
    }
}
template <int HD, int KIND, typename FR>
__device__ __forceinline__ float g1_v(const FR& f, int t, int j) {
    if constexpr (KIND == KV_F32) {
        const float4& x = f.v[t][j >> 2];
        return (j & 3) == 0 ? x.x : (j & 3) == 1 ? x.y : (j & 3) == 2 ? x.z : x.w;
    } else {
        return (float)f.v[t][j];
    }
}

// One 32-key block folded into the wave's running (m, l, o) for its one
// query: qv holds the lane's query dims 32s + 8grp + j, already in log2-score
// units; o[t] is this lane's context sum for dim 16t + col over keys 8grp ..
// of every block; m and l are wave-uniform. pw: the wave's 32-float LDS row.
template <int HD, int KIND, bool MASK, typename FR>
__device__ __forceinline__ void fold_block_g1(const FR& f, const float (&qv)[HD / 32][8], int p0, int tk, int col,
                                              int grp, float& m_run, float& l_run, float (&o)[HD / 16],
                                              float* pw) {
    constexpr int NS = HD / 32, NT = HD / 16;
    float sc[2];
#pragma unroll
    for (int T = 0; T < 2; ++T) {
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = __builtin_fmaf(g1_k<HD, KIND>(f, T, s, j), qv[s][j], acc);
        acc = sum4grp(acc);
        if constexpr (MASK) {
            const int key = p0 + 8 * (col >> 2) + 4 * T + (col & 3);
            acc = key < tk ? acc : ninf();
        }
        sc[T] = acc;
    }
    const float mx = wave_max(fmaxf(sc[0], sc[1]));
    const float mn = fmaxf(m_run, mx);
    const float fac = ex2(m_run - mn);
    m_run = mn;
    const float e0 = ex2(sc[0] - mn), e1 = ex2(sc[1] - mn);
    // Each key's probability sits in the four grp lanes of its column: the
    // wave sum is four times the block's (an exact scaling).
    l_run = l_run * fac + wave_sum(e0 + e1) * 0.25f;
    if (__any(fac != 1.0f)) {
#pragma unroll
        for (int t = 0; t < NT; ++t) o[t] *= fac;
    }
    if (grp == 0) {
        pw[8 * (col >> 2) + (col & 3)] = e0;
        pw[8 * (col >> 2) + 4 + (col & 3)] = e1;
    }
    __builtin_amdgcn_wave_barrier();
    const float4 pa = *reinterpret_cast<const float4*>(pw + 8 * grp);
    const float4 pb = *reinterpret_cast<const float4*>(pw + 8 * grp + 4);
    const float pp[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float acc = o[t];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float v = g1_v<HD, KIND>(f, t, j);
            // A cache may hold non-finite garbage past tk: 0 * NaN is NaN.
            if constexpr (MASK) v = p0 + 8 * grp + j < tk ? v : 0.0f;
            acc = __builtin_fmaf(pp[j], v, acc);
        }
        o[t] = acc;
    }
    __builtin_amdgcn_wave_barrier();  // the row is read before the next block's writes
}

// The hardware id of the XCD this wave runs on (HW_REG_XCC_ID, bits 3:0).
__device__ __forceinline__ unsigned xcc_id() { return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15u; }

// Arrival counter (64 bits, on its own 256-byte line): bits 0-15 count the
// arrivals, bits 16-31 sum the arriving workgroups' XCC ids x and bits 32-47
// their squares. The n arrivals shared one XCD exactly when n * sum(x^2) =
// sum(x)^2 (Cauchy-Schwarz equality). Ids are < 16 and splits <= 256, so no
// field overflows into the next.
__device__ __forceinline__ unsigned long long arrival(unsigned x) {
    return 1ull | ((unsigned long long)x << 16) | ((unsigned long long)(x * x) << 32);
}
__device__ __forceinline__ bool one_xcd(unsigned long long c) {
    const unsigned long long n = c & 0xffff, s1 = (c >> 16) & 0xffff, s2 = (c >> 32) & 0xffff;
    return n * s2 == s1 * s1;
}

template <int HD, int KIND, int VA, bool G1>
__global__ __launch_bounds__(DT, KIND == KV_F32 ? 1 : 2) void attn_decode_kernel(DecodeArgs a) {
    constexpr int NS = HD / 32;
    constexpr int NT = HD / 16;
    constexpr bool TILED = KIND == KV_T16 || KIND == KV_TQ8;
    constexpr int OBW = 16 * (HD + 4);  // one wave's O^T in LDS, [column][dim], padded
    __shared__ float lds[DW * OBW];
    __shared__ float wm[DW][16], wl[DW][16], gl[16];
    __shared__ int last;
    __shared__ __attribute__((aligned(16))) float prow[DW][32];  // G1: a block's probabilities
    static_assert(!G1 || KIND != KV_TQ8, "the Q8_0 cache decodes through the MFMA path");
    // G1L: the f32 cache at head_dim 64 in line order (FragF32L).
    constexpr bool G1L = G1 && KIND == KV_F32 && HD == 64;
    using FR = std::conditional_t<G1L, FragF32L<HD>,
                                  std::conditional_t<G1 && KIND == KV_F32, FragF32<HD>, Frag<HD, KIND>>>;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    int split = blockIdx.x, h = blockIdx.y, seq = blockIdx.z;
    const int nit = a.nit;
    if (a.xcd) {
        const int item = (int)(blockIdx.x % 8) * a.grid8 + (int)(blockIdx.x / 8);
        split = item % a.splits;
        h = (item / a.splits) % a.kv_heads;
        seq = item / (a.splits * a.kv_heads);
    }
    const int group = a.group;
    const int tk = a.tk_arr ? min(a.tk_arr[seq], a.tk) : a.tk;
    const int slot = a.slot_arr ? a.slot_arr[seq] : 0;
    if (a.slot_arr && (slot < 0 || slot >= a.slots || tk <= 0)) {
        // A sequence the batch describes wrongly gets NaN, never a read
        // outside its cache.
        if (split == 0)
            for (int e = tid; e < group * HD; e += DT)
                a.out[a.out_off + (size_t)seq * a.out_stride + (size_t)h * group * HD + e] = __builtin_nanf("");
        return;
    }
    const int span = DW * nit * 32;
    const int nsplit = (tk + span - 1) / span;
    if (split >= nsplit) return;  // whole workgroup: a shorter sequence of the batch

    Ctx c;
    c.tk = tk;
    c.cap = a.cap;
    const size_t kvh = (size_t)slot * a.kv_heads + h;
    if constexpr (TILED) {
        c.bstride = KIND == KV_T16 ? 2L * 32 * HD * 2 : tq8_block_bytes(HD);
        c.k = reinterpret_cast<const char*>(a.k) + kvh * (size_t)tiled_nblk(a.cap) * c.bstride;
        c.v = nullptr;
    } else {
        constexpr int esz = KIND == KV_F32 ? 4 : 2;
        c.bstride = 0;
        c.k = reinterpret_cast<const char*>(a.k) + kvh * a.cap * HD * esz;
        c.v = reinterpret_cast<const char*>(a.v) + kvh * HD * a.cap * esz;
    }

    // This wave's blocks: b_i = first + i * DW for i < nb, through a two-deep
    // pipeline (block i+1's loads in flight while block i is folded). The
    // context's partial last block, when it is this wave's, is its last (nf
    // full blocks, then it): every block is loaded the same way, and only the
    // partial one is folded with the mask. The first blocks' loads go out
    // before the queries are read.
    const int first = split * DW * nit + wave;
    const int nfull = tk >> 5;
    const int nf = nfull > first ? min(nit, (nfull - first + DW - 1) / DW) : 0;
    const bool tail = (tk & 31) && nfull >= first && (nfull - first) % DW == 0 && (nfull - first) / DW < nit;
    // Tiled caches keep the partial block out of the pipeline (loaded and
    // folded after it): with it inside, the pipeline's epilogue needs both
    // fold variants for both register sets, which cost the tiled decode
    // ~0.05 us (C2 9.39 -> 9.44 us) for a gain only partial blocks see.
    constexpr bool TP = !TILED;  // the partial block inside the pipeline
    const int nb = nf + (TP && tail ? 1 : 0);
    FR f0, f1;
    auto ld = [&](int p, FR& f) __attribute__((always_inline)) {
        if constexpr (G1L) load_block_f32l<HD, VA>(c, p, lane, f);
        else if constexpr (G1 && KIND == KV_F32) load_block_f32v<HD, VA>(c, p, lane, f);
        else load_block<HD, KIND, VA, !G1>(c, p, lane, f);
    };
    // The first two blocks go out before the queries are read: the queries'
    // first use waits for every load issued before them, so a block issued
    // after that would start a second memory round trip.
    if (nb > 0) ld(first * 32, f0);
    if (nb > 1 && !(KIND == KV_F32 && HD == 128)) ld((first + DW) * 32, f1);

    // The group's queries as B operands, hi + lo (columns past the group are
    // read from column 0 and zeroed, so every load is unconditional). The
    // score scale and log2(e) ride on the query, so a product is already a
    // log2-unit score.
    const float* q = a.q + a.q_off + (size_t)seq * a.q_stride + ((size_t)h * group) * HD;
    const bool qok = col < group;
    const float* qc = q + (size_t)(qok ? col : 0) * HD + 8 * grp;
    float ql4[4];  // G1L: the query's dims 4 (lane%16) .. +3, log2-score units
    if constexpr (G1L) {
        const float4 x = *reinterpret_cast<const float4*>(q + 4 * (lane & 15));
        const float f = a.qscale * a.score_l2;
        ql4[0] = x.x * f;
        ql4[1] = x.y * f;
        ql4[2] = x.z * f;
        ql4[3] = x.w * f;
    }
    float4 qx[NS][2];
#pragma unroll
    for (int s = 0; s < NS && !G1L; ++s) {
        qx[s][0] = reinterpret_cast<const float4*>(qc + 32 * s)[0];
        qx[s][1] = reinterpret_cast<const float4*>(qc + 32 * s)[1];
    }
    half8 qh[NS], ql[NS];
    float qv[NS][8];  // G1: the query in f32, log2-score units
#pragma unroll
    for (int s = 0; s < NS && !G1L; ++s) {
        const float x[8] = {qx[s][0].x, qx[s][0].y, qx[s][0].z, qx[s][0].w,
                            qx[s][1].x, qx[s][1].y, qx[s][1].z, qx[s][1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if constexpr (G1) {
                qv[s][j] = x[j] * a.qscale * a.score_l2;
            } else {
                half_t hh, ll;
                split_h(qok ? x[j] * a.qscale * a.score_l2 : 0.0f, hh, ll);
                qh[s][j] = hh;
                ql[s][j] = ll;
            }
        }
    }

    float m_run = ninf(), l_run = 0.0f;
    floatx4 o[NT];
    float o1[NT];  // G1: lane's context sums for dims 16t + col
    float ol[8];   // G1L: lane's context sums for dims 8i + lane/8
#pragma unroll
    for (int i = 0; i < 8; ++i) ol[i] = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        o[t] = zero_f4();
        o1[t] = 0.0f;
    }
    auto fold = [&](const FR& f, int p, auto mask_tag) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask_tag)::value;
        if constexpr (G1L)
            fold_block_g1l<HD, MASK>(f, ql4, p, tk, lane, m_run, l_run, ol, prow[wave]);
        else if constexpr (G1)
            fold_block_g1<HD, KIND, MASK>(f, qv, p, tk, col, grp, m_run, l_run, o1, prow[wave]);
        else
            fold_block<HD, KIND, MASK>(f, qh, ql, p, tk, grp, a.score_l2, m_run, l_run, o);
    };

    // Two blocks in flight: while block i is folded, block i + 1 is on its
    // way. Inside the loop every prefetch is unconditional (a block past this
    // wave's last is clamped to its last and re-read, at most once per wave
    // and only for an odd block count), so the wait counter stands at the
    // same count on every path into a fold and each fold waits only for its
    // own block. The scheduling barriers keep each prefetch ahead of the fold
    // it is meant to overlap (left alone, the scheduler sinks loads towards
    // their uses).
    // f32 caches at head_dim 128: one block in flight (two would not fit in
    // the register file and would spill to scratch).
    constexpr bool DEEP = !(KIND == KV_F32 && HD == 128);
    // Block j of the wave, folded with the mask when it is the partial one.
    auto fold_j = [&](const FR& f, int j) __attribute__((always_inline)) {
        const int p = (first + j * DW) * 32;
        if (TP && tail && j == nf) fold(f, p, std::true_type{});
        else fold(f, p, std::false_type{});
    };
    int i = 0;
    if constexpr (!DEEP) {
        for (; i < nb; ++i) {
            if (i > 0) ld((first + i * DW) * 32, f0);
            fold_j(f0, i);
        }
    }
    // Blocks i, i + 1 are full here (only the last block can be partial).
    for (; DEEP && i + 2 < nb; i += 2) {
        const int p0 = (first + i * DW) * 32;
        const int p1 = (first + (i + 1) * DW) * 32;
        const int p2 = (first + (i + 2) * DW) * 32;
        const int p3 = (first + min(i + 3, nb - 1) * DW) * 32;
        fold(f0, p0, std::false_type{});
        __builtin_amdgcn_sched_barrier(0);
        ld(p2, f0);
        __builtin_amdgcn_sched_barrier(0);
        fold(f1, p1, std::false_type{});
        __builtin_amdgcn_sched_barrier(0);
        ld(p3, f1);
        __builtin_amdgcn_sched_barrier(0);
    }
    // The last one or two blocks (already in f0, f1).
    if (DEEP && i < nb) fold_j(f0, i);
    if (DEEP && i + 1 < nb) fold_j(f1, i + 1);
    if (!TP && tail) {
        ld(nfull * 32, f0);
        fold(f0, nfull * 32, std::true_type{});
    }
    float olc = 0.0f;
    if constexpr (G1L) {
        olc = g1l_context(ol, lane);
    } else if constexpr (G1) {
        // A wave with no block keeps m = -inf, l = 0, o = 0 (weight 0 below).
#pragma unroll
        for (int t = 0; t < NT; ++t) o1[t] = sum4grp(o1[t]);
    } else {
        l_run = sum4grp(l_run);
    }

    // Combine the four waves: each wave leaves its (m, l) and its unscaled
    // O^T in LDS ([query column][dim], 16-byte writes), one barrier, and the
    // combining reads weight wave w by 2^(m_w - M), M = max_w m_w.
    if (grp == 0) {
        wm[wave][col] = m_run;
        wl[wave][col] = l_run;
    }
    float* ob = lds + wave * OBW;
    if constexpr (G1L) {
        ob[8 * (lane & 7) + (lane >> 3)] = olc;
    } else if constexpr (G1) {
        if (grp == 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t) ob[16 * t + col] = o1[t];
        }
    } else {
#pragma unroll
        for (int t = 0; t < NT; ++t)
            *reinterpret_cast<floatx4*>(&ob[col * (HD + 4) + 16 * t + 4 * grp]) = o[t];
    }
    __syncthreads();
    // Wave weights of query column g, and its combined normaliser.
    auto weights = [&](int g, float (&f)[DW]) {
        float M = ninf();
#pragma unroll
        for (int w = 0; w < DW; ++w) M = fmaxf(M, wm[w][g]);
#pragma unroll
        for (int w = 0; w < DW; ++w) f[w] = wm[w][g] == ninf() ? 0.0f : ex2(wm[w][g] - M);
        return M;
    };

    float* out = a.out + a.out_off + (size_t)seq * a.out_stride;
    int8_t* tc = nullptr;
    float* ts = nullptr;
    if (a.twin_codes) {
        const size_t oo = a.out_off + (size_t)seq * a.out_stride;
        tc = a.twin_codes + oo;
        ts = a.twin_scales + (oo >> 5);
    }
    const int n = group * HD;
    if (nsplit == 1) {
        for (int e = tid; e < n; e += DT) {
            const int g = e / HD, d = e % HD;
            float f[DW];
            weights(g, f);
            float acc = 0.0f, L = 0.0f;
#pragma unroll
            for (int w = 0; w < DW; ++w) {
                acc += lds[w * OBW + g * (HD + 4) + d] * f[w];
                L += wl[w][g] * f[w];
            }
            emit(out, tc, ts, (size_t)h * group * HD + e, acc / L);
        }
        return;
    }

    // Publish this split's partial: O [g][HD] (relative to its own max) in
    // the O area, (m, l) per g in the ML area, 16 bytes a store.
    const size_t head = (size_t)seq * a.kv_heads + h;
    float* po = a.part + (head * a.splits) * n;
    float* pml = a.part + a.ml_off + head * a.ml_stride;
    auto partial4 = [&](int e4) __attribute__((always_inline)) {
        const int g = (4 * e4) / HD, d = (4 * e4) % HD;
        float f[DW];
        weights(g, f);
        floatx4 acc = zero_f4();
#pragma unroll
        for (int w = 0; w < DW; ++w) acc += *reinterpret_cast<const floatx4*>(&lds[w * OBW + g * (HD + 4) + d]) * f[w];
        return acc;
    };
    auto ml = [&](int g) __attribute__((always_inline)) {
        float f[DW];
        const float M = weights(g, f);
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < DW; ++w) L += wl[w][g] * f[w];
        return floatx4{M, L, 0.0f, 0.0f};
    };
    if (a.two_phase) {
        // A separate merge launch follows: plain stores, and done.
        for (int e4 = tid; e4 < n / 4; e4 += DT)
            *reinterpret_cast<floatx4*>(po + (size_t)split * n + 4 * e4) = partial4(e4);
        if (tid < group) {
            const floatx4 x = ml(tid);
            pml[((size_t)split * group + tid) * 2] = x[0];
            pml[((size_t)split * group + tid) * 2 + 1] = x[1];
        }
        return;
    }
    // Cross-workgroup hand-off without cache-wide fences: the partial is
    // stored, the stores are waited for, and only then is the arrival
    // counted; the last arriver reads the partials. Across XCDs the stores
    // and the merger's loads are agent-scope (coherent past the XCDs'
    // separate L2s); with a head's splits all on one XCD (a.xcd) plain
    // stores into the shared L2 and L2 reads suffice. A release/acquire
    // fence pair would write back and invalidate the whole L2 of the XCD on
    // every workgroup, which measured several times the cost of the
    // attention itself.
    const bool loc = a.xcd != 0;
    {
        const __amdgpu_buffer_rsrc_t rp =
            __builtin_amdgcn_make_buffer_rsrc(po + (size_t)split * n, 0, n * 4, 0x00020000);
        typedef float v4 __attribute__((ext_vector_type(4)));
        for (int e4 = tid; e4 < n / 4; e4 += DT) {
            const floatx4 x = partial4(e4);
            const v4 y = {x[0], x[1], x[2], x[3]};
            if (loc) __builtin_amdgcn_raw_buffer_store_b128(y, rp, e4 * 16, 0, 0);
            else __builtin_amdgcn_raw_buffer_store_b128(y, rp, e4 * 16, 0, AUX_AGENT);
        }
    }
    if (tid < group) {
        const floatx4 x = ml(tid);
        float* d = pml + ((size_t)split * group + tid) * 2;
        if (loc) {
            d[0] = x[0];
            d[1] = x[1];
        } else {
            st_coherent(d, x[0]);
            st_coherent(d + 1, x[1]);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    unsigned long long* ctr = reinterpret_cast<unsigned long long*>(a.ctr + head * CTR_STRIDE);
    if (tid == 0) {
        const unsigned x = a.xcd_fake ? (blockIdx.x / 8) % 8 : xcc_id();
        const unsigned long long add = arrival(x);
        const unsigned long long prev = __hip_atomic_fetch_add(ctr, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // 1: the last arrival, every partial readable here; 2: the last
        // arrival of an XCD-local head whose workgroups did not share an XCD.
        last = (prev & 0xffff) != (unsigned long long)(nsplit - 1) ? 0 : (a.xcd && !one_xcd(prev + add)) ? 2 : 1;
    }
    __syncthreads();
    if (!last) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (last == 2) {
        // Partials stored into another XCD's L2 are not visible here: the
        // head's context is reported as NaN (its twin with NaN scales).
        for (int e = tid; e < n; e += DT) {
            const size_t idx = (size_t)h * group * HD + e;
            out[idx] = __builtin_nanf("");
            if (tc) {
                tc[idx] = 0;
                if ((e & 31) == 0) ts[idx >> 5] = __builtin_nanf("");
            }
        }
        if (tid == 0) {
            __hip_atomic_store(ctr, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (a.lost) __hip_atomic_store(a.lost, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        return;
    }
    if (loc) merge_head<HD, AUX_XCD>(po, pml, nsplit, group, lds, gl, out, tc, ts, (size_t)h * group * HD);
    else merge_head<HD, AUX_AGENT>(po, pml, nsplit, group, lds, gl, out, tc, ts, (size_t)h * group * HD);
    if (tid == 0) __hip_atomic_store(ctr, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The merge of one head's splits as a launch of its own, after a two-phase
// attention launch: one workgroup per (sequence, kv head).
template <int HD>
__global__ __launch_bounds__(DT) void attn_merge_kernel(DecodeArgs a) {
    __shared__ float lds[4096];
    __shared__ float gl[16];
    const int h = blockIdx.x, seq = blockIdx.y;
    const int group = a.group;
    const int tk = a.tk_arr ? min(a.tk_arr[seq], a.tk) : a.tk;
    const int slot = a.slot_arr ? a.slot_arr[seq] : 0;
    if (a.slot_arr && (slot < 0 || slot >= a.slots || tk <= 0)) return;
    const int nit = a.nit;
    const int span = DW * nit * 32;
    const int nsplit = (tk + span - 1) / span;
    if (nsplit <= 1) return;  // the attention launch wrote this head itself
    const int n = group * HD;
    const size_t head = (size_t)seq * a.kv_heads + h;
    const float* po = a.part + (head * a.splits) * n;
    const float* pml = a.part + a.ml_off + head * a.ml_stride;
    float* out = a.out + a.out_off + (size_t)seq * a.out_stride;
    int8_t* tc = nullptr;
    float* ts = nullptr;
    if (a.twin_codes) {
        const size_t oo = a.out_off + (size_t)seq * a.out_stride;
        tc = a.twin_codes + oo;
        ts = a.twin_scales + (oo >> 5);
    }
    merge_head<HD, 0>(po, pml, nsplit, group, lds, gl, out, tc, ts, (size_t)h * group * HD);
}

// ------------------------------------------------------------------------
// Stream-K batched decode over a tiled cache (the device-planned batch).
//
// Every (sequence, kv head, 32-key block) of the batch is one position of a
// flat list, sequence-major, then kv head, then block; the launch's waves
// each take a contiguous range of it of equal cost (its blocks, plus one
// block's worth for each kv head starting in it: a segment's start and end
// cost a wave about a block's time), so every wave streams about the same
// work whatever the spread of the sequences' lengths (a per-head split of a
// fixed span leaves the last, short split of each head idle for most of the
// launch). A wave walks its range with the two-deep
// block prefetch of attn_decode_kernel; the range falls into segments, one
// per kv head it touches:
//   - a segment that is a whole head: the wave normalises and writes the
//     context rows itself;
//   - a segment that is part of a head (at most the first and the last of
//     the range): the wave publishes (m, l, O) to its own partial slot
//     (slot 0: a segment ending before the range does; slot 1: the one
//     ending with it) and, after its range, counts its arrival at the head;
//     the last arriver merges the head's partials in range order.
// A segment's queries are moved into LDS by a direct-to-LDS load issued just
// before its first block's loads, so they arrive with that block and cost
// no registers while in flight.

// Lane l's value as a wave-uniform (scalar) one: l must be uniform.
__device__ __forceinline__ int rdlane(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ long rdlane64(long v, int l) {
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)((unsigned long)v >> 32), l);
    return (long)(((unsigned long)hi << 32) | lo);
}
__device__ __forceinline__ long rdfirst64(long v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((int)(uint32_t)((unsigned long)v >> 32));
    return (long)(((unsigned long)hi << 32) | lo);
}

// The batch's sequences, one per lane (nseq <= 64): blocks per kv head and
// the position of the sequence's first block in the flat list.
struct SkSeqs {
    int nb;      // 32-key blocks per kv head (0: a sequence the batch describes wrongly)
    int tk, slot;
    long base;   // flat position of (this sequence, kv head 0, block 0)
    long total;  // positions in the whole batch (wave-uniform)
    long vbase;  // the same in cost units (see sk_first)
    long vend;   // vbase of the next sequence
    long vtotal; // cost units of the whole batch (wave-uniform)
};
__device__ __forceinline__ SkSeqs sk_seqs(const DecodeArgs& a, int lane) {
    SkSeqs q;
    q.tk = 0;
    q.slot = 0;
    q.nb = 0;
    if (lane < a.nseq) {
        q.tk = min(a.tk_arr[lane], a.tk);
        q.slot = a.slot_arr[lane];
        if (q.slot >= 0 && q.slot < a.slots && q.tk > 0) q.nb = (q.tk + 31) >> 5;
    }
    const long cnt = (long)q.nb * a.kv_heads;
    long incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const long y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    q.base = incl - cnt;
    q.total = rdlane64(incl, 63);
    // Cost units: a kv head costs its blocks plus one for the segment that
    // starts at it (its queries converted, a context written or a partial
    // stashed: about one block's time in a wave's stream).
    const long vcnt = q.nb > 0 ? (long)(q.nb + 1) * a.kv_heads : 0;
    long vincl = vcnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const long y = __shfl_up(vincl, o, 64);
        if (lane >= o) vincl += y;
    }
    q.vbase = vincl - vcnt;
    q.vend = vincl;
    q.vtotal = rdlane64(vincl, 63);
    return q;
}

// The partition of the flat block list over the nw waves that take part
// (nw <= total), balanced in cost units: each kv head is one unit (its
// start) followed by its blocks, and wave u takes the blocks whose units
// lie in [u V / nw, (u + 1) V / nw), V = vtotal. Wave u's range of blocks is
// [sk_first(u), sk_first(u + 1)); it is empty when its units hold only a
// head's start.
__device__ __forceinline__ long sk_first(const SkSeqs& q, long u, long nw) {
    const long x = u * q.vtotal / nw;
    if (x >= q.vtotal) return q.total;
    // The sequence holding unit x: those ending at or before it are a
    // prefix of the lanes (lanes past the batch end at V > x).
    const int s = __popcll(__ballot(q.vend <= x));
    const int nb = rdlane(q.nb, s);
    const long xo = x - rdlane64(q.vbase, s);
    const long h = xo / (nb + 1), j = xo % (nb + 1);
    return rdlane64(q.base, s) + h * nb + (j > 0 ? j - 1 : 0);
}
// The wave whose range holds block p.
__device__ __forceinline__ long sk_owner(const SkSeqs& q, long p, int kv_heads, long nw) {
    const int s = __popcll(__ballot(q.base + (long)q.nb * kv_heads <= p));
    const int nb = rdlane(q.nb, s);
    const long off = p - rdlane64(q.base, s);
    const long v = rdlane64(q.vbase, s) + off + off / nb + 1;
    return ((v + 1) * nw - 1) / q.vtotal;
}

// Where flat position p lies: sequence, kv head, block (all wave-uniform).
struct SkPos {
    int s, h, blk, nb, tk, slot;
};
__device__ __forceinline__ SkPos sk_locate(const SkSeqs& q, long p, int kv_heads) {
    // Sequences whose blocks all lie before p (a prefix of the lanes: lanes
    // past the batch have base = total > p).
    const int s = __popcll(__ballot(q.base + (long)q.nb * kv_heads <= p));
    SkPos r;
    r.s = s;
    r.nb = rdlane(q.nb, s);
    r.tk = rdlane(q.tk, s);
    r.slot = rdlane(q.slot, s);
    const long off = p - rdlane64(q.base, s);
    r.h = (int)(off / r.nb);
    r.blk = (int)(off % r.nb);
    return r;
}

// s_waitcnt with only the vector-memory count bounded (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// The LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// One tiled Q8_0 block from LDS (at byte address b) into a fragment set, as
// one asm block that also waits for its own reads. The compiler cannot tell
// which direct-to-LDS load wrote which bytes, so before an LDS read it knows
// of it waits for every outstanding load, the next block's prefetch
// included; this read is ordered by the caller's explicit vmcnt wait instead.
template <int HD>
__device__ __forceinline__ void ring_read(uint32_t b, int lane, int grp, Frag<HD, KV_TQ8>& f);
template <>
__device__ __forceinline__ void ring_read<128>(uint32_t b, int lane, int grp, Frag<128, KV_TQ8>& f) {
    // codes: K (T, sp) at ((T*2 + sp)*64 + lane)*16, V tile pair tp at 4096 + (tp*64 + lane)*16;
    // scales: K dim block i at 8192 + (i*4 + grp)*16, V at 8192 + 256 + ...
    const uint32_t c = b + 16 * lane, sc = b + 8192 + 16 * grp;
    asm volatile(
        "ds_read_b128 %0, %16\n"
        "ds_read_b128 %1, %16 offset:1024\n"
        "ds_read_b128 %2, %16 offset:2048\n"
        "ds_read_b128 %3, %16 offset:3072\n"
        "ds_read_b128 %4, %16 offset:4096\n"
        "ds_read_b128 %5, %16 offset:5120\n"
        "ds_read_b128 %6, %16 offset:6144\n"
        "ds_read_b128 %7, %16 offset:7168\n"
        "ds_read_b128 %8, %17\n"
        "ds_read_b128 %9, %17 offset:64\n"
        "ds_read_b128 %10, %17 offset:128\n"
        "ds_read_b128 %11, %17 offset:192\n"
        "ds_read_b128 %12, %17 offset:256\n"
        "ds_read_b128 %13, %17 offset:320\n"
        "ds_read_b128 %14, %17 offset:384\n"
        "ds_read_b128 %15, %17 offset:448\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(f.kc[0][0]), "=&v"(f.kc[0][1]), "=&v"(f.kc[1][0]), "=&v"(f.kc[1][1]), "=&v"(f.vc[0]), "=&v"(f.vc[1]),
          "=&v"(f.vc[2]), "=&v"(f.vc[3]), "=&v"(f.ks[0]), "=&v"(f.ks[1]), "=&v"(f.ks[2]), "=&v"(f.ks[3]), "=&v"(f.vs[0]),
          "=&v"(f.vs[1]), "=&v"(f.vs[2]), "=&v"(f.vs[3])
        : "v"(c), "v"(sc));
}
template <>
__device__ __forceinline__ void ring_read<64>(uint32_t b, int lane, int grp, Frag<64, KV_TQ8>& f) {
    // codes: K (T, 0) at (T*64 + lane)*16, V tile pair tp at 2048 + (tp*64 + lane)*16;
    // scales: K dim block i at 4096 + (i*4 + grp)*16, V at 4096 + 128 + ...
    const uint32_t c = b + 16 * lane, sc = b + 4096 + 16 * grp;
    asm volatile(
        "ds_read_b128 %0, %8\n"
        "ds_read_b128 %1, %8 offset:1024\n"
        "ds_read_b128 %2, %8 offset:2048\n"
        "ds_read_b128 %3, %8 offset:3072\n"
        "ds_read_b128 %4, %9\n"
        "ds_read_b128 %5, %9 offset:64\n"
        "ds_read_b128 %6, %9 offset:128\n"
        "ds_read_b128 %7, %9 offset:192\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(f.kc[0][0]), "=&v"(f.kc[1][0]), "=&v"(f.vc[0]), "=&v"(f.vc[1]), "=&v"(f.ks[0]), "=&v"(f.ks[1]),
          "=&v"(f.vs[0]), "=&v"(f.vs[1])
        : "v"(c), "v"(sc));
}

// A lane's query operands from a raw [g][HD] f32 buffer in LDS (b = the
// byte address of its column's dims 8*grp ..): dims 32s + 8grp + 0..7 as
// two float4 per s, read as one asm block (see ring_read). Every output of
// these multi-read blocks is early-clobber ("=&v"): the reads are issued
// back to back, so an output sharing a register with the address would be
// overwritten by one read's return while a later read still needs it.
template <int HD>
__device__ __forceinline__ void q_read(uint32_t b, float4 (&x)[HD / 32][2]);
template <>
__device__ __forceinline__ void q_read<128>(uint32_t b, float4 (&x)[4][2]) {
    asm volatile(
        "ds_read_b128 %0, %8\n"
        "ds_read_b128 %1, %8 offset:16\n"
        "ds_read_b128 %2, %8 offset:128\n"
        "ds_read_b128 %3, %8 offset:144\n"
        "ds_read_b128 %4, %8 offset:256\n"
        "ds_read_b128 %5, %8 offset:272\n"
        "ds_read_b128 %6, %8 offset:384\n"
        "ds_read_b128 %7, %8 offset:400\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(x[0][0]), "=&v"(x[0][1]), "=&v"(x[1][0]), "=&v"(x[1][1]), "=&v"(x[2][0]), "=&v"(x[2][1]), "=&v"(x[3][0]),
          "=&v"(x[3][1])
        : "v"(b));
}
template <>
__device__ __forceinline__ void q_read<64>(uint32_t b, float4 (&x)[2][2]) {
    asm volatile(
        "ds_read_b128 %0, %4\n"
        "ds_read_b128 %1, %4 offset:16\n"
        "ds_read_b128 %2, %4 offset:128\n"
        "ds_read_b128 %3, %4 offset:144\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(x[0][0]), "=&v"(x[0][1]), "=&v"(x[1][0]), "=&v"(x[1][1])
        : "v"(b));
}

// The Q8_0 stream-K kernel. Each wave owns one LDS slot of a whole tiled
// block, filled by direct-to-LDS loads (no registers held while a block is
// in flight): fold i waits for the slot, reads block i into registers,
// refills the slot with block i + 1 and folds from registers. The wave is
// busy most of a block's period (the loads' issue, the LDS read and the
// fold), so a deeper ring only adds bytes in flight, and more bytes in flight
// than one block per wave measured slower (two-slot ring 58.9 vs 58.6 us,
// three-slot slower again). One workgroup per compute unit: at two, 2048
// concurrent streams measured slower (first data up to 17 us late).
template <int HD>
__global__ __launch_bounds__(DT, 1) void attn_decode_sk_kernel(DecodeArgs a) {
    constexpr int W = DW;
    constexpr int RING = 1;
    constexpr int KIND = KV_TQ8;
    constexpr int NS = HD / 32;
    constexpr int NT = HD / 16;
    constexpr int BB = (int)tq8_block_bytes(HD);  // bytes of one block
    constexpr int CODE_I = 64 * HD / 1024;        // 1 KB code loads per block
    constexpr int SCL_L = (BB - 64 * HD) / 16;    // lanes of the one scale load
    constexpr int LPB = CODE_I + 1;               // load instructions per block
    static_assert(SCL_L <= 64, "scales in one wave-wide load");
    __shared__ __attribute__((aligned(16))) char ring[W][RING][BB];
    // The LDS budget: the ring plus the largest query buffers the host
    // launches with (two of group <= 16 rows of HD floats per wave).
    static_assert(W == SK_WAVES && BB == (int)sk_block_bytes(HD), "the host's LDS arithmetic");
    static_assert(sizeof(ring) + sk_qdyn_max(HD) <= SK_LDS_MAX, "stream-K LDS over a workgroup's 160 KB");
    // Dynamic: per wave, one raw query buffer of group * HD floats (the
    // destination of a segment's direct-to-LDS query loads).
    extern __shared__ __attribute__((aligned(16))) float sk_qraw[];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, grp = lane >> 4;
    const int group = a.group, kv = a.kv_heads;
    const int n = group * HD;           // context floats per (sequence, kv head)
    const long heads_n = (long)kv * n;  // context floats per sequence

    const SkSeqs sq = sk_seqs(a, lane);
    const long total = sq.total;
    const long nw = min((long)a.items * W, total);
    const long u = (long)blockIdx.x * W + wave;

    // A sequence the batch describes wrongly gets a NaN row (written by the
    // launch's first wave), never a read outside its cache.
    if (u == 0) {
        for (int s = 0; s < a.nseq; ++s) {
            if (rdlane(sq.nb, s) == 0) {
                float* o = a.out + a.out_off + (size_t)s * a.out_stride;
                for (long e = lane; e < heads_n; e += 64) o[e] = __builtin_nanf("");
            }
        }
    }
    if (u >= nw) return;
    const long p_first = sk_first(sq, u, nw), p_end = sk_first(sq, u + 1, nw);
    if (p_first >= p_end) return;  // units holding only a head's start
    const long nblk_cap = tiled_nblk(a.cap);

    // The next block to issue, as a cursor stepping through the list
    // (wave-uniform, no division per block).
    SkPos ci = sk_locate(sq, p_first, kv);
    auto step = [&](SkPos& r) {
        if (++r.blk < r.nb) return;
        r.blk = 0;
        if (++r.h < kv) return;
        r.h = 0;
        do {
            ++r.s;
        } while (r.s < 63 && rdlane(sq.nb, r.s) == 0);
        r.nb = rdlane(sq.nb, r.s);
        r.tk = rdlane(sq.tk, r.s);
        r.slot = rdlane(sq.slot, r.s);
    };
    // A segment's queries, raw f32 [g][HD], are moved into one of the wave's
    // two LDS query buffers just before its first block's loads, so they
    // land with that block. Segments take the buffers alternately, in issue
    // order; by the time a third segment's queries are issued, the first's
    // have been converted (a fold converts its segment's queries before it
    // issues the block two ahead).
    float* const qbufs = sk_qraw + (size_t)wave * 2 * n;
    int q_in = 0, q_out = 0;  // the buffer the next segment's queries go to / come from
    auto load_q = [&](const SkPos& r, int buf) {
        const float* src = a.q + a.q_off + (size_t)r.s * a.q_stride + (size_t)r.h * n;
        for (int i = 0; i < n; i += 256)
            if (i + 4 * lane < n) __builtin_amdgcn_global_load_lds(src + i + 4 * lane, qbufs + buf * n + i, 16, 0, 0);
    };
    // Vector-memory instructions this wave has issued (loads and stores
    // retire in issue order on this part), and the count just after each
    // ring slot's block: a fold waits with vmcnt = everything issued since.
    // Every instruction counted here is issued with lane 0 active.
    int vm_ops = 0, mark[RING] = {};
    const int q_instr = (n + 255) / 256;
    // Issues the block at the cursor into ring slot `slot` and returns where
    // it lies; past the range's end nothing is issued. The first block of a
    // segment is preceded by its queries' loads.
    long pi = p_first;
    auto issue = [&](int slot) {
        const SkPos r = ci;
        if (pi >= p_end) return r;
        if (pi == p_first || r.blk == 0) {
            load_q(r, q_in);
            vm_ops += q_instr;
            q_in ^= 1;
        }
        char* dst = &ring[wave][slot][0];
        // One buffer resource over the (slot, kv head)'s blocks; the block
        // offset and the 1 KB steps are scalar, so the loads cost no VALU.
        const int hs_i = __builtin_amdgcn_readfirstlane(r.slot * kv + r.h);
        const char* hbase = reinterpret_cast<const char*>(a.k) + (size_t)hs_i * (size_t)nblk_cap * BB;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char*>(hbase), 0, (int)(nblk_cap * BB), 0x00020000);
        const int soff = __builtin_amdgcn_readfirstlane(r.blk) * BB;
        // The instruction's immediate offset would move the LDS address as
        // well as the global one: the 1 KB steps go into the scalar offset.
        const int vo = 16 * lane;
#pragma unroll
        for (int i = 0; i < CODE_I; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst + 1024 * i, 16, vo, soff + 1024 * i, 0, AUX_STREAM);
        static_assert(CODE_I == 4 || CODE_I == 8, "code loads per block");
        if (lane < SCL_L)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst + 64 * HD, 16, 16 * lane, soff + 64 * HD, 0, AUX_STREAM);
        vm_ops += LPB;
        mark[slot] = vm_ops;
        if (pi + 1 < p_end) step(ci);
        ++pi;
        return r;
    };

    half8 qh[NS], ql[NS];
    float m_run = ninf(), l_run = 0.0f;
    floatx4 o[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] = zero_f4();  // finite from the start (see the segment start)
    // Pending partial publications (slot 0, slot 1): the head's flat start
    // position, or -1.
    long pend0 = -1, pend1 = -1;

    // A partial of a head, O [g][HD] and (m, l) [g], into this wave's slot sl
    // with agent-scope (coherent) stores.
    auto publish = [&](int sl, const floatx4 (&ov)[NT], float m, float l) __attribute__((always_inline)) {
        const size_t slot_i = (size_t)u * 2 + sl;
        float* po = a.part + slot_i * (16 * HD);
        float* pml = a.part + a.ml_off + slot_i * 32;
        const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(po, 0, 16 * HD * 4, 0x00020000);
        typedef float v4 __attribute__((ext_vector_type(4)));
        if (col < group) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
                __builtin_amdgcn_raw_buffer_store_b128(v4{ov[t][0], ov[t][1], ov[t][2], ov[t][3]}, rp,
                                                       (col * HD + 16 * t + 4 * grp) * 4, 0, 16);  // sc1
            if (grp == 0) {
                typedef float v2 __attribute__((ext_vector_type(2)));
                const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(pml, 0, 128, 0x00020000);
                __builtin_amdgcn_raw_buffer_store_b64(v2{m, l}, rm, 8 * col, 0, 16);  // sc1
            }
        }
    };
    // The range's first segment when it is part of a head.
    floatx4 o0[NT];
    float m_first = 0.0f, l_first = 0.0f;

    SkPos rs[RING];
#pragma unroll
    for (int i = 0; i < RING; ++i) rs[i] = issue(i);

    // Fold of the block in ring slot `slot` at flat position pp; rn: the
    // position of the block issued into the slot afterwards.
    auto fold_at = [&](int slot, long pp, const SkPos r, SkPos& rn) {
        // This block has landed once at most the instructions issued after
        // its loads are outstanding: nothing, or a whole head's context
        // stores (rounded down; a smaller count only waits longer).
        const int after = __builtin_amdgcn_readfirstlane(vm_ops - mark[slot]);
        if (after >= NT) wait_vm<NT>();
        else wait_vm<0>();
        Frag<HD, KIND> f;
        ring_read<HD>(lds_addr(&ring[wave][slot][0]), lane, grp, f);
        if (pp == p_first || r.blk == 0) {
            // A new segment: its queries as hi + lo f16 B operands, scaled
            // into log2 units.
            const bool qok = col < group;
            float4 x[NS][2];
            q_read<HD>(lds_addr(qbufs + q_out * n) + 4 * ((qok ? col : 0) * HD + 8 * grp), x);
            q_out ^= 1;
            const float qs = qok ? a.qscale * a.score_l2 : 0.0f;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const float xs[8] = {x[s][0].x, x[s][0].y, x[s][0].z, x[s][0].w,
                                     x[s][1].x, x[s][1].y, x[s][1].z, x[s][1].w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    half_t hh, ll;
                    split_h(xs[j] * qs, hh, ll);
                    qh[s][j] = hh;
                    ql[s][j] = ll;
                }
            }
            // The previous segment's context is already written: with m at
            // -inf the fold's rescale factor 2^(m - M) is exactly 0 and
            // clears o (always finite). An explicit reset here made the
            // compiler carry o through AGPRs, 64 moves a block.
            m_run = ninf();
            l_run = 0.0f;
        }
        // The slot (and the query buffer) are read: refill the slot with the
        // next block.
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        rn = issue(slot);
        if (r.blk == r.nb - 1 && (r.tk & 31))
            fold_block_q8<HD, true>(f, qh, ql, r.blk * 32, r.tk, grp, m_run, l_run, o);
        else
            fold_block_q8<HD, false>(f, qh, ql, r.blk * 32, r.tk, grp, m_run, l_run, o);
        // The end of a segment: a head's last block, or the range's.
        if (r.blk == r.nb - 1 || pp == p_end - 1) {
            const float lsum = sum4grp(l_run);
            // A whole head: its block 0 lies in this range too.
            if (r.blk == r.nb - 1 && pp - r.blk >= p_first) {
                if (col < group) {
                    float* out = a.out + a.out_off + (size_t)r.s * a.out_stride + (size_t)r.h * n + (size_t)col * HD;
                    const float inv = 1.0f / lsum;
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        *reinterpret_cast<floatx4*>(out + 16 * t + 4 * grp) = o[t] * inv;
                }
                vm_ops += NT;
            } else {
                // Part of a head. The range's last segment is published at
                // once (the range ends here); its first one is kept in
                // registers and published after the range: a store here
                // would hold every later block's wait (vector-memory
                // operations retire in issue order) for its write-through.
                const long hs = rdlane64(sq.base, r.s) + (long)r.h * r.nb;
                if (pp == p_end - 1) {
                    publish(1, o, m_run, lsum);
                    pend1 = hs;
                } else {
#pragma unroll
                    for (int t = 0; t < NT; ++t) o0[t] = o[t];
                    m_first = m_run;
                    l_first = lsum;
                    pend0 = hs;
                }
            }
        }
    };

    for (long p = p_first; p < p_end; p += RING) {
#pragma unroll
        for (int i = 0; i < RING; ++i) {
            if (p + i >= p_end) break;
            fold_at(i, p + i, rs[i], rs[i]);
        }
    }

    if (pend0 >= 0) publish(0, o0, m_first, l_first);
    // Arrivals: after every partial store has completed, count this wave at
    // each head it published part of (at most two), both atomics in one round
    // trip; the last arriver at a head merges it.
    __builtin_amdgcn_s_waitcnt(0);
    pend0 = rdfirst64(pend0);
    pend1 = rdfirst64(pend1);
    struct Head {
        long c0, c1;  // its contributors, in range order
        int last_sl;  // the last contributor's slot for it
        int idx;      // sequence * kv + kv head
    };
    auto head_at = [&](long hs) {
        const SkPos r = sk_locate(sq, hs, kv);
        const long he = hs + r.nb;
        Head h;
        h.c0 = sk_owner(sq, hs, kv, nw);
        h.c1 = sk_owner(sq, he - 1, kv, nw);
        // Every contributor but the last publishes the head as the segment
        // ending its range (slot 1); the last one, as slot 1 only if its
        // range ends with the head.
        h.last_sl = sk_first(sq, h.c1 + 1, nw) == he ? 1 : 0;
        h.idx = r.s * kv + r.h;
        h.c0 = rdfirst64(h.c0);
        h.c1 = rdfirst64(h.c1);
        h.last_sl = __builtin_amdgcn_readfirstlane(h.last_sl);
        h.idx = __builtin_amdgcn_readfirstlane(h.idx);
        return h;
    };
    Head h0 = head_at(pend0 >= 0 ? pend0 : 0), h1 = head_at(pend1 >= 0 ? pend1 : 0);
    unsigned prev0 = 0, prev1 = 0;
    if (lane == 0) {
        if (pend0 >= 0)
            prev0 = __hip_atomic_fetch_add(a.ctr + (size_t)h0.idx * CTR_STRIDE, 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
        if (pend1 >= 0)
            prev1 = __hip_atomic_fetch_add(a.ctr + (size_t)h1.idx * CTR_STRIDE, 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    }
    // Lane 0's counts (the whole wave is active), kept in scalar registers
    // so the merge's addressing stays wave-uniform.
    prev0 = __builtin_amdgcn_readfirstlane(prev0);
    prev1 = __builtin_amdgcn_readfirstlane(prev1);
    const bool m0 = pend0 >= 0 && prev0 == (unsigned)(h0.c1 - h0.c0);
    const bool m1 = pend1 >= 0 && prev1 == (unsigned)(h1.c1 - h1.c0);
    if (!m0 && !m1) return;
    // The heads to merge: A, then B when there are two.
    const int nm_all = (int)m0 + (int)m1;
    const Head A0 = m0 ? h0 : h1, B0 = h1;
    auto slot_of = [&](const Head& h, long c) -> size_t {
        return (size_t)c * 2 + (c < h.c1 ? 1 : h.last_sl);
    };
    // A head of at most KF contributors and a context of at most 512 floats
    // is merged straight from registers: every contributor's O columns and
    // (m, l) pairs are loaded at once (both heads' together), then, per head
    // and in range order, M = max m, w = 2^(m - M), l = sum w l, O = sum w O.
    // Which path a head takes depends on the head alone, and the two heads'
    // arithmetic never mixes, so a head's bits do not depend on the wave
    // that merges it or on what it merges beside.
    constexpr int KF = 10;
    const bool fit = n <= 512;
    const bool fa = fit && A0.c1 - A0.c0 + 1 <= KF, fb = fit && nm_all > 1 && B0.c1 - B0.c0 + 1 <= KF;
    if (fa || fb) {
        const Region pr = region(a.part, (uint32_t)((a.ml_off + (long)a.items * W * 2 * 32) * 4));
        const Head F0 = fa ? A0 : B0, F1 = B0;
        const int nf = (int)fa + (int)fb;
        const int c0n = (int)(F0.c1 - F0.c0 + 1), c1n = nf > 1 ? (int)(F1.c1 - F1.c0 + 1) : 0;
        int e4[2], g[2];
        bool on[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            e4[j] = lane + 64 * j;
            on[j] = e4[j] < n / 4;
            g[j] = on[j] ? (4 * e4[j]) / HD : 0;
        }
        floatx4 ov[2][KF][2];
        float2 mv[2][KF][2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const Head& H = hh ? F1 : F0;
            const int cn = hh ? c1n : c0n;
#pragma unroll
            for (int k = 0; k < KF; ++k) {
                if (k < cn) {
                    const uint32_t si = (uint32_t)__builtin_amdgcn_readfirstlane((int)slot_of(H, H.c0 + k));
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const float4 x = ld_region4<AUX_AGENT>(pr, (si * (16 * HD) + 4 * (on[j] ? e4[j] : 0)) * 4);
                        ov[hh][k][j] = floatx4{x.x, x.y, x.z, x.w};
                        mv[hh][k][j] = ld_region2<AUX_AGENT>(pr, (uint32_t)(a.ml_off + si * 32 + 2 * g[j]) * 4);
                    }
                }
            }
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            if (hh >= nf) continue;
            const Head& H = hh ? F1 : F0;
            const int cn = hh ? c1n : c0n;
            float* out = a.out + a.out_off + (size_t)(H.idx / kv) * a.out_stride + (size_t)(H.idx % kv) * n;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float M = ninf();
#pragma unroll
                for (int k = 0; k < KF; ++k)
                    if (k < cn) M = fmaxf(M, mv[hh][k][j].x);
                float L = 0.0f;
                floatx4 acc = zero_f4();
#pragma unroll
                for (int k = 0; k < KF; ++k) {
                    if (k < cn) {
                        const float w = ex2(mv[hh][k][j].x - M);
                        L = __builtin_fmaf(mv[hh][k][j].y, w, L);
                        acc[0] = __builtin_fmaf(ov[hh][k][j][0], w, acc[0]);
                        acc[1] = __builtin_fmaf(ov[hh][k][j][1], w, acc[1]);
                        acc[2] = __builtin_fmaf(ov[hh][k][j][2], w, acc[2]);
                        acc[3] = __builtin_fmaf(ov[hh][k][j][3], w, acc[3]);
                    }
                }
                if (on[j]) *reinterpret_cast<floatx4*>(out + 4 * e4[j]) = acc * (1.0f / L);
            }
        }
    }
    // The heads left to the general merge.
    const bool ga = !fa, gb = nm_all > 1 && !fb;
    const int nm = (int)ga + (int)gb;
    const Head A = ga ? A0 : B0, B = B0;
    const long cntA = nm ? A.c1 - A.c0 + 1 : 0, cntB = nm > 1 ? B.c1 - B.c0 + 1 : 0;
    // The general merge (heads of more than KF contributors, or contexts of
    // more than 512 floats). Each head's contributors are merged, in range order, in chunks of KC
    // counted from the head's first: a chunk's (m, l) pairs go straight into
    // LDS (half of the wave's idle ring per head, lane-strided dword loads),
    // its max M is taken once, and every contributor then adds 2^(m - M)
    // times its l and O. The arithmetic of a head depends only on its own
    // contributors, never on which wave merges it or what it merges beside.
    // O moves in batches of 8 contributors (both heads' chunks as one list),
    // two float4 loads each, under the 63 vector-memory instructions a wave
    // can have outstanding.
    // Lane owns float4 e4 = lane + 64 j of a head's [g][HD] context.
    constexpr int HALF_F = ((RING * BB / 4 - 64) / 2) / 64 * 64;  // floats of LDS per head
    const int gp = 2 * group;                            // (m, l) floats per contributor
    const int KC = HALF_F / gp;
    float* const mls = reinterpret_cast<float*>(&ring[wave][0][0]);
    float* const Ms = mls + 2 * HALF_F;  // [head][16]: the chunk's running max per query head
    const float* const mlp = a.part + a.ml_off;
    for (int j0 = 0; nm > 0 && j0 * 64 < n / 4; j0 += 2) {
        int e4[2], g[2];
        bool on[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            e4[j] = lane + 64 * (j0 + j);
            on[j] = e4[j] < n / 4;
            g[j] = on[j] ? (4 * e4[j]) / HD : 0;
        }
        float M[2][2] = {{ninf(), ninf()}, {ninf(), ninf()}}, L[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
        floatx4 acc[2][2] = {{zero_f4(), zero_f4()}, {zero_f4(), zero_f4()}};
        for (long t0 = 0; t0 < cntA || t0 < cntB; t0 += KC) {
            const int nA = (int)max(0L, min((long)KC, cntA - t0)), nB = (int)max(0L, min((long)KC, cntB - t0));
            const int nc = nA + nB;
            // The previous chunk's LDS reads are done before it is overwritten.
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const Head& h = hh ? B : A;
                const int nh = hh ? nB : nA;
                for (int i = 0; i * 64 < nh * gp; ++i) {
                    const int fi = 64 * i + lane, k = fi / gp;
                    // Lanes past the chunk read a harmless float (slot 0's).
                    const float* src = mlp + (k < nh ? slot_of(h, h.c0 + t0 + k) * 32 + fi % gp : 0);
                    __builtin_amdgcn_global_load_lds(src, mls + hh * HALF_F + 64 * i, 4, 0, AUX_AGENT);
                }
            }
            auto batch = [&](auto mbc, int cb) __attribute__((always_inline)) {
                constexpr int MB = decltype(mbc)::value;
                float4 ov[MB][2];
#pragma unroll
                for (int k = 0; k < MB; ++k) {
                    const int e = cb + k;
                    const bool live = e < nc, inB = e >= nA;
                    // Wave-uniform: kept scalar so the load needs no waterfall.
                    const size_t si = (unsigned)__builtin_amdgcn_readfirstlane(
                        (int)(!live ? 0 : inB ? slot_of(B, B.c0 + t0 + (e - nA)) : slot_of(A, A.c0 + t0 + e)));
                    const Region ro = region(a.part + si * (16 * HD), live ? 16 * HD * 4 : 0);
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        ov[k][j] = ld_region4<AUX_AGENT>(ro, (uint32_t)(on[j] ? e4[j] * 16 : 0));
                }
                wait_vm<0>();
                if (cb == 0) {
                    // The chunk's max per head and column (reads clamped to
                    // the chunk: repeats do not move a max), then the running
                    // sums rescaled to it.
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int nh = hh ? nB : nA;
                        if (nh == 0) continue;
                        const float* ml = mls + hh * HALF_F;
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            float bm = ninf();
                            for (int c = 0; c < nh; c += 8) {
                                float x[8];
#pragma unroll
                                for (int q = 0; q < 8; ++q) x[q] = ml[min(c + q, nh - 1) * gp + 2 * g[j]];
#pragma unroll
                                for (int q = 0; q < 8; ++q) bm = fmaxf(bm, x[q]);
                            }
                            const float mn = fmaxf(M[hh][j], bm);
                            const float al = ex2(M[hh][j] - mn);
                            M[hh][j] = mn;
                            L[hh][j] *= al;
                            acc[hh][j] = acc[hh][j] * al;
                            if (on[j] && (4 * e4[j]) % HD == 0) Ms[hh * 16 + g[j]] = mn;
                        }
                    }
                    // The chunk's (m, l) pairs become (w, l w), w = 2^(m - M),
                    // in place, one pair per lane: one exponential per pair
                    // rather than per lane and contributor.
                    for (int i = lane; i < nc * group; i += 64) {
                        const int k = i / group, gg = i % group, hh = k >= nA ? 1 : 0;
                        float2* pr = reinterpret_cast<float2*>((hh ? mls + HALF_F + (k - nA) * gp : mls + k * gp) + 2 * gg);
                        const float2 v = *pr;
                        const float w = ex2(v.x - Ms[hh * 16 + gg]);
                        *pr = make_float2(w, v.y * w);
                    }
                }
                float2 mv[MB][2];
#pragma unroll
                for (int k = 0; k < MB; ++k) {
                    const int e = min(cb + k, nc - 1);
                    const float* ml = e >= nA ? mls + HALF_F + (e - nA) * gp : mls + e * gp;
#pragma unroll
                    for (int j = 0; j < 2; ++j) mv[k][j] = *reinterpret_cast<const float2*>(ml + 2 * g[j]);
                }
                // Explicit fmaf: the rounding is the same in either batch
                // size. Which head a contributor adds to is a wave-uniform
                // branch with fixed register indices (an index chosen at run
                // time would put the accumulators in scratch).
                auto add = [&](floatx4(&ac)[2], float(&Lh)[2], int k) __attribute__((always_inline)) {
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const float w = mv[k][j].x;
                        Lh[j] += mv[k][j].y;
                        ac[j][0] = __builtin_fmaf(ov[k][j].x, w, ac[j][0]);
                        ac[j][1] = __builtin_fmaf(ov[k][j].y, w, ac[j][1]);
                        ac[j][2] = __builtin_fmaf(ov[k][j].z, w, ac[j][2]);
                        ac[j][3] = __builtin_fmaf(ov[k][j].w, w, ac[j][3]);
                    }
                };
                // Head A's contributors come first in the list, B's after.
                const int kA = min(MB, nA - cb), kn = min(MB, nc - cb);
#pragma unroll
                for (int k = 0; k < MB; ++k)
                    if (k < kA) add(acc[0], L[0], k);
#pragma unroll
                for (int k = 0; k < MB; ++k)
                    if (k >= kA && k < kn) add(acc[1], L[1], k);
            };
            // Batches of 8 contributors: their O registers (64 VGPRs) stay
            // under the stream loop's own need, so the kernel keeps one
            // register budget (a batch of 24 set it, with spills).
            for (int cb = 0; cb < nc; cb += 8) batch(std::integral_constant<int, 8>{}, cb);
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            if (hh >= nm) continue;
            const int hi = hh ? B.idx : A.idx;
            float* out = a.out + a.out_off + (size_t)(hi / kv) * a.out_stride + (size_t)(hi % kv) * n;
#pragma unroll
            for (int j = 0; j < 2; ++j)
                if (on[j]) *reinterpret_cast<floatx4*>(out + 4 * e4[j]) = acc[hh][j] * (1.0f / L[hh][j]);
        }
    }
    if (lane == 0) {
        __hip_atomic_store(a.ctr + (size_t)A0.idx * CTR_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (nm_all > 1)
            __hip_atomic_store(a.ctr + (size_t)B0.idx * CTR_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

#define DECODE_INST(HD, KIND, VA, G1) template __global__ void attn_decode_kernel<HD, KIND, VA, G1>(DecodeArgs);
#define DECODE_INST2(HD, KIND, VA) DECODE_INST(HD, KIND, VA, false) DECODE_INST(HD, KIND, VA, true)
DECODE_INST2(64, KV_F16, 16) DECODE_INST2(128, KV_F16, 16) DECODE_INST2(64, KV_F16, 8) DECODE_INST2(128, KV_F16, 8)
DECODE_INST2(64, KV_F32, 16) DECODE_INST2(128, KV_F32, 16) DECODE_INST2(64, KV_F32, 8)
DECODE_INST2(128, KV_F32, 8) DECODE_INST2(64, KV_T16, 16) DECODE_INST2(128, KV_T16, 16)
DECODE_INST(64, KV_TQ8, 16, false) DECODE_INST(128, KV_TQ8, 16, false)

template __global__ void attn_decode_sk_kernel<64>(DecodeArgs);
template __global__ void attn_decode_sk_kernel<128>(DecodeArgs);
template __global__ void attn_merge_kernel<64>(DecodeArgs);
template __global__ void attn_merge_kernel<128>(DecodeArgs);

static hipError_t launch_merge(int hd, const DecodeArgs& a, int kv_heads, int nseq, hipStream_t st) {
    dim3 grid(kv_heads, nseq), block(DT);
    if (hd == 64) hipLaunchKernelGGL((attn_merge_kernel<64>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((attn_merge_kernel<128>), grid, block, 0, st, a);
    return hipGetLastError();
}

static hipError_t launch_attn(int hd, int kind, const DecodeArgs& a, int kv_heads, int nseq, hipStream_t st) {
    if (a.sk) {
        dim3 grid(a.items), block(DT);
        if (kind != KV_TQ8 || !(hd == 64 || hd == 128)) return hipErrorInvalidValue;
        // The raw query buffers; with the static ring, never over a
        // workgroup's LDS (the entry point refuses larger groups first).
        const size_t qdyn = sk_qdyn_bytes(hd, a.group);
        if (sk_lds_bytes(hd, a.group) > SK_LDS_MAX) return hipErrorInvalidValue;
        if (hd == 128) hipLaunchKernelGGL((attn_decode_sk_kernel<128>), grid, block, qdyn, st, a);
        else hipLaunchKernelGGL((attn_decode_sk_kernel<64>), grid, block, qdyn, st, a);
        return hipGetLastError();
    }
    const dim3 grid = a.xcd ? dim3(a.splits * kv_heads * nseq) : dim3(a.splits, kv_heads, nseq);
    dim3 block(DT);
    DecodeArgs b = a;
    b.grid8 = (int)(grid.x / 8);
    const int esz = kind == KV_F32 ? 4 : 2;
    const int va = (kind == KV_T16 || kind == KV_TQ8) ? 16 : (((long)a.cap * esz) % 16 == 0 ? 16 : 8);
    // Group 1 (MHA) folds on the VALU.
    const bool g1 = a.group == 1 && kind != KV_TQ8 && !getenv("LLMTIE_DECODE_G1_MFMA");
#define L(HD, KIND, VA, G1)                                                                    \
    if (hd == HD && kind == KIND && va == VA && g1 == G1) {                                    \
        hipLaunchKernelGGL((attn_decode_kernel<HD, KIND, VA, G1>), grid, block, 0, st, b);      \
        return hipGetLastError();                                                              \
    }
#define L2(HD, KIND, VA) L(HD, KIND, VA, false) L(HD, KIND, VA, true)
    L2(64, KV_F16, 16) L2(128, KV_F16, 16) L2(64, KV_F16, 8) L2(128, KV_F16, 8)
    L2(64, KV_F32, 16) L2(128, KV_F32, 16) L2(64, KV_F32, 8) L2(128, KV_F32, 8)
    L2(64, KV_T16, 16) L2(128, KV_T16, 16) L(64, KV_TQ8, 16, false) L(128, KV_TQ8, 16, false)
#undef L2
#undef L
    return hipErrorInvalidValue;
}

__global__ void fill_u32_kernel(unsigned* p, size_t n, unsigned v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

hipError_t launch_fill_u32(unsigned* p, size_t n, unsigned v, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(fill_u32_kernel, dim3(blocks), dim3(256), 0, st, p, n, v);
    return hipGetLastError();
}

hipError_t launch_decode(int hd, int kind, const DecodeArgs& a, int kv_heads, int nseq, hipStream_t st) {
    hipError_t e = launch_attn(hd, kind, a, kv_heads, nseq, st);
    if (e != hipSuccess || a.sk || !a.two_phase || a.splits <= 1) return e;
    return launch_merge(hd, a, kv_heads, nseq, st);
}

}  // namespace llmtie
