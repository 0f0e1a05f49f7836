// Split-K single-token decode attention for gfx950.
//
// Replaces the reference's `attn_decode_impl` / `attn_decode_run_impl` /
// `ad_publish_merge` (crates/llmtie-cuda/src/kernels.rs:5779-6505) with one
// MFMA kernel, templated on the head width and on the cache's storage:
//   KV_F16 - K [kv][cap][hd] f16, V [kv][hd][cap] f16 (the reference layout)
//   KV_F32 - the same layout at f32 (the Whisper decoder's self cache)
//   KV_Q8  - GGUF Q8_0 blocks (32 int8 codes + one f16 scale per 32 dims of a
//            position): K codes [slot][kv][cap][hd], V codes transposed
//            [slot][kv][hd][cap], scales of both [slot][kv][cap][hd/32].
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
#include "common.h"
#include "decode.h"

namespace llmtie {

constexpr int DW = 4;              // waves per workgroup
constexpr int DT = DW * LLMTIE_WAVE;  // threads per workgroup

template <int HD, int KIND>
struct Frag;

template <int HD>
struct Frag<HD, KV_F16> {
    half8 k[2][HD / 32];
    half8 v[HD / 16];
};
template <int HD>
struct Frag<HD, KV_F32> {
    half8 kh[2][HD / 32], kl[2][HD / 32];
    half8 vh[HD / 16], vl[HD / 16];
};
template <int HD>
struct Frag<HD, KV_Q8> {
    half8 k[2][HD / 32];
    half8 v[HD / 16];
    half_t dk[8][HD / 32];  // scales of keys 8*grp + j, block b
    half_t dv[8][HD / 32];
};

struct Ctx {
    const char* k;   // this (sequence, kv head)'s K base (codes or values)
    const char* v;   // V^T base
    const uint16_t* ks;  // Q8 scales of K, row of key 0
    const uint16_t* vs;
    int tk, cap;
    bool v16;  // V rows are 16-byte aligned at every 8-key boundary
};

template <int HD, int KIND>
__device__ __forceinline__ void load_block(const Ctx& c, int p0, int col, int grp, Frag<HD, KIND>& f) {
    constexpr int NS = HD / 32;
    constexpr int NT = HD / 16;
    // Keys.
#pragma unroll
    for (int T = 0; T < 2; ++T) {
        const int key = p0 + 8 * (col >> 2) + 4 * T + (col & 3);
        const bool ok = key < c.tk;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int d0 = 32 * s + 8 * grp;
            if constexpr (KIND == KV_F16) {
                f.k[T][s] = ok ? ld_h8(c.k + ((size_t)key * HD + d0) * 2) : zero_h8();
            } else if constexpr (KIND == KV_F32) {
                half8 h = zero_h8(), l = zero_h8();
                if (ok) {
                    const float4* p = reinterpret_cast<const float4*>(c.k + ((size_t)key * HD + d0) * 4);
                    const float4 a = p[0], b = p[1];
                    const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        half_t hh, ll;
                        split_h(x[j], hh, ll);
                        h[j] = hh;
                        l[j] = ll;
                    }
                }
                f.kh[T][s] = h;
                f.kl[T][s] = l;
            } else {
                f.k[T][s] = ok ? ld_q8x8(reinterpret_cast<const int8_t*>(c.k) + (size_t)key * HD + d0) : zero_h8();
            }
        }
    }
    // Values: V^T rows d = 16t + col, keys p0 + 8*grp + 0..7.
    const int kb = p0 + 8 * grp;
    const bool full = kb + 8 <= c.tk;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const size_t row = (size_t)(16 * t + col) * c.cap + kb;
        if constexpr (KIND == KV_F16) {
            const uint16_t* p = reinterpret_cast<const uint16_t*>(c.v) + row;
            if (full) {
                f.v[t] = c.v16 ? ld_h8(p) : ld_h8_a4(p);
            } else {
                half8 h = zero_h8();
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (kb + j < c.tk) h[j] = __builtin_bit_cast(half_t, p[j]);
                f.v[t] = h;
            }
        } else if constexpr (KIND == KV_F32) {
            const float* p = reinterpret_cast<const float*>(c.v) + row;
            float x[8];
            if (full) {
                if (c.v16) {
                    const float4 a = reinterpret_cast<const float4*>(p)[0];
                    const float4 b = reinterpret_cast<const float4*>(p)[1];
                    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
                    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
                } else {
#pragma unroll
                    for (int j = 0; j < 8; j += 2) {
                        const float2 a = reinterpret_cast<const float2*>(p + j)[0];
                        x[j] = a.x;
                        x[j + 1] = a.y;
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = (kb + j < c.tk) ? p[j] : 0.0f;
            }
            half8 h, l;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                half_t hh, ll;
                split_h(x[j], hh, ll);
                h[j] = hh;
                l[j] = ll;
            }
            f.vh[t] = h;
            f.vl[t] = l;
        } else {
            const int8_t* p = reinterpret_cast<const int8_t*>(c.v) + row;
            if (full) {
                f.v[t] = ld_q8x8(p);
            } else {
                half8 h = zero_h8();
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (kb + j < c.tk) h[j] = (half_t)(float)p[j];
                f.v[t] = h;
            }
        }
    }
    if constexpr (KIND == KV_Q8) {
        // Scales of keys kb .. kb + 7, every block: 8 * HD/32 contiguous halves.
        constexpr int NB = HD / 32;
        const uint16_t* ks = c.ks + (size_t)kb * NB;
        const uint16_t* vs = c.vs + (size_t)kb * NB;
        if (full) {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                // 16 bytes = 8 halves = keys 2i, 2i+1 (NB == 4) or 4i..4i+3 (NB == 2)
                const half8 a = ld_h8(ks + 8 * i);
                const half8 b = ld_h8(vs + 8 * i);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    f.dk[(8 * i + e) / NB][(8 * i + e) % NB] = a[e];
                    f.dv[(8 * i + e) / NB][(8 * i + e) % NB] = b[e];
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const bool ok = kb + j < c.tk;
                    f.dk[j][b] = ok ? __builtin_bit_cast(half_t, ks[j * NB + b]) : (half_t)0.0f;
                    f.dv[j][b] = ok ? __builtin_bit_cast(half_t, vs[j * NB + b]) : (half_t)0.0f;
                }
        }
    }
}

// One 32-key block folded into the wave's running softmax state.
template <int HD, int KIND>
__device__ __forceinline__ void fold_block(const Frag<HD, KIND>& f, const half8 (&qh)[HD / 32],
                                           const half8 (&ql)[HD / 32], int p0, int tk, int grp,
                                           float score_l2, float& m_run, float& l_run,
                                           floatx4 (&o)[HD / 16]) {
    constexpr int NS = HD / 32;
    constexpr int NT = HD / 16;
    float sc[8];
#pragma unroll
    for (int T = 0; T < 2; ++T) {
        floatx4 acc = zero_f4();
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            if constexpr (KIND == KV_F16) {
                acc = mfma16(f.k[T][s], qh[s], acc);
                acc = mfma16(f.k[T][s], ql[s], acc);
            } else if constexpr (KIND == KV_F32) {
                acc = mfma16(f.kh[T][s], qh[s], acc);
                acc = mfma16(f.kh[T][s], ql[s], acc);
                acc = mfma16(f.kl[T][s], qh[s], acc);
            } else {
                floatx4 b = mfma16(f.k[T][s], qh[s], zero_f4());
                b = mfma16(f.k[T][s], ql[s], b);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] += (float)f.dk[4 * T + r][s] * b[r];
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[4 * T + r] = acc[r];
    }
    const int kb = p0 + 8 * grp;
    float mx = ninf();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sc[j] = (kb + j < tk) ? sc[j] * score_l2 : ninf();
        mx = fmaxf(mx, sc[j]);
    }
    mx = max4grp(mx);
    const float mn = fmaxf(m_run, mx);
    const float fac = ex2(m_run - mn);
    m_run = mn;
    float p[8], ps = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        p[j] = ex2(sc[j] - mn);
        ps += p[j];
    }
    l_run = l_run * fac + ps;
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] *= fac;

    if constexpr (KIND == KV_Q8) {
        constexpr int NB = HD / 32;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            half8 ph, pl;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                half_t hh, ll;
                split_h(p[j] * (float)f.dv[j][b], hh, ll);
                ph[j] = hh;
                pl[j] = ll;
            }
#pragma unroll
            for (int t = 2 * b; t < 2 * b + 2; ++t) {
                o[t] = mfma16(f.v[t], ph, o[t]);
                o[t] = mfma16(f.v[t], pl, o[t]);
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
            if constexpr (KIND == KV_F16) {
                o[t] = mfma16(f.v[t], ph, o[t]);
                o[t] = mfma16(f.v[t], pl, o[t]);
            } else {
                o[t] = mfma16(f.vh[t], ph, o[t]);
                o[t] = mfma16(f.vh[t], pl, o[t]);
                o[t] = mfma16(f.vl[t], ph, o[t]);
            }
        }
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

template <int HD, int KIND>
__global__ __launch_bounds__(DT) void attn_decode_kernel(DecodeArgs a) {
    constexpr int NS = HD / 32;
    constexpr int NT = HD / 16;
    constexpr int OBS = HD * 17;  // one wave's O^T in LDS, padded
    __shared__ float lds[DW * OBS > 16 * DECODE_MAX_SPLITS ? DW * OBS : 16 * DECODE_MAX_SPLITS];
    __shared__ float wm[DW][16], wl[DW][16], gm[16], gl[16];
    __shared__ int last;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int split = blockIdx.x, h = blockIdx.y, seq = blockIdx.z;
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
    const int span = DW * a.nit * 32;
    const int nsplit = (tk + span - 1) / span;
    if (split >= nsplit) return;  // whole workgroup: a shorter sequence of the batch

    Ctx c;
    c.tk = tk;
    c.cap = a.cap;
    const size_t kvh = (size_t)slot * a.kv_heads + h;
    const int esz = KIND == KV_F32 ? 4 : (KIND == KV_F16 ? 2 : 1);
    c.k = reinterpret_cast<const char*>(a.k) + kvh * a.cap * HD * esz;
    c.v = reinterpret_cast<const char*>(a.v) + kvh * HD * a.cap * esz;
    c.ks = a.ks ? a.ks + kvh * a.cap * (HD / 32) : nullptr;
    c.vs = a.vs ? a.vs + kvh * a.cap * (HD / 32) : nullptr;
    c.v16 = ((a.cap * esz) & 15) == 0;

    // The group's queries as B operands, hi + lo.
    const float* q = a.q + a.q_off + (size_t)seq * a.q_stride + ((size_t)h * group) * HD;
    half8 qh[NS], ql[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        half8 hv = zero_h8(), lv = zero_h8();
        if (col < group) {
            const float4* p = reinterpret_cast<const float4*>(q + (size_t)col * HD + 32 * s + 8 * grp);
            const float4 x0 = p[0], x1 = p[1];
            const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                half_t hh, ll;
                split_h(x[j] * a.qscale, hh, ll);
                hv[j] = hh;
                lv[j] = ll;
            }
        }
        qh[s] = hv;
        ql[s] = lv;
    }

    float m_run = ninf(), l_run = 0.0f;
    floatx4 o[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] = zero_f4();

    // Blocks of this wave: p(i) = split*span + (i*DW + wave)*32, i < nit.
    const int base = split * span + wave * 32;
    Frag<HD, KIND> f0, f1;
    if (base < tk) load_block<HD, KIND>(c, base, col, grp, f0);
    for (int i = 0; i < a.nit; i += 2) {
        const int p0 = base + i * DW * 32;
        const int p1 = p0 + DW * 32;
        const int p2 = p1 + DW * 32;
        if (p0 >= tk) break;
        const bool has1 = i + 1 < a.nit && p1 < tk;
        const bool has2 = i + 2 < a.nit && p2 < tk;
        if (has1) load_block<HD, KIND>(c, p1, col, grp, f1);
        fold_block<HD, KIND>(f0, qh, ql, p0, tk, grp, a.score_l2, m_run, l_run, o);
        if (has2) load_block<HD, KIND>(c, p2, col, grp, f0);
        if (has1) fold_block<HD, KIND>(f1, qh, ql, p1, tk, grp, a.score_l2, m_run, l_run, o);
    }
    l_run = sum4grp(l_run);

    // Combine the four waves: M = max m_w, each wave's O scaled by 2^(m_w - M).
    if (grp == 0) {
        wm[wave][col] = m_run;
        wl[wave][col] = l_run;
    }
    __syncthreads();
    float M = ninf();
#pragma unroll
    for (int w = 0; w < DW; ++w) M = fmaxf(M, wm[w][col]);
    const float myf = (m_run == ninf()) ? 0.0f : ex2(m_run - M);
    float* ob = lds + wave * OBS;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) ob[(16 * t + 4 * grp + r) * 17 + col] = o[t][r] * myf;
    if (tid < 16) {
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < DW; ++w) {
            const float mw = wm[w][tid];
            L += (mw == ninf()) ? 0.0f : wl[w][tid] * ex2(mw - M);
        }
        gm[tid] = M;
        gl[tid] = L;
    }
    __syncthreads();

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
            float acc = 0.0f;
#pragma unroll
            for (int w = 0; w < DW; ++w) acc += lds[w * OBS + d * 17 + g];
            emit(out, tc, ts, (size_t)h * group * HD + e, acc / gl[g]);
        }
        return;
    }

    // Publish this split's partial: [g][HD] O (relative to its own max), m, l.
    const size_t rec = (size_t)(HD + 2);
    const size_t head_part = (((size_t)seq * gridDim.y + h) * a.splits) * group * rec;
    float* mine = a.part + head_part + (size_t)split * group * rec;
    for (int e = tid; e < n; e += DT) {
        const int g = e / HD, d = e % HD;
        float acc = 0.0f;
#pragma unroll
        for (int w = 0; w < DW; ++w) acc += lds[w * OBS + d * 17 + g];
        mine[g * rec + d] = acc;
    }
    if (tid < group) {
        mine[tid * rec + HD] = gm[tid];
        mine[tid * rec + HD + 1] = gl[tid];
    }
    __threadfence();
    __syncthreads();
    unsigned* ctr = a.ctr + (size_t)seq * gridDim.y + h;
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last = prev == (unsigned)(nsplit - 1);
    }
    __syncthreads();
    if (!last) return;
    __threadfence();

    // The merge, in split order. Per group: a wave finds the max and the
    // weights 2^(m_s - M) (kept in LDS), and the sum L.
    const float* all = a.part + head_part;
    float* wts = lds;  // [16][DECODE_MAX_SPLITS]
    __syncthreads();   // everyone is done reading `lds` as O^T
    for (int g = wave; g < group; g += DW) {
        float mx = ninf();
        for (int s = lane; s < nsplit; s += 64) {
            const float ms = all[((size_t)s * group + g) * rec + HD];
            mx = fmaxf(mx, ms);
        }
#pragma unroll
        for (int o2 = 32; o2 > 0; o2 >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o2, 64));
        float L = 0.0f;
        for (int s = lane; s < nsplit; s += 64) {
            const float* pc = all + ((size_t)s * group + g) * rec;
            const float w = ex2(pc[HD] - mx);
            wts[g * DECODE_MAX_SPLITS + s] = w;
            L += pc[HD + 1] * w;
        }
        // Fixed-order sum across lanes: butterfly is order-deterministic.
#pragma unroll
        for (int o2 = 32; o2 > 0; o2 >>= 1) L += __shfl_xor(L, o2, 64);
        if (lane == 0) gl[g] = L;
    }
    __syncthreads();
    for (int e = tid; e < n; e += DT) {
        const int g = e / HD, d = e % HD;
        float acc = 0.0f;
        for (int s = 0; s < nsplit; ++s)
            acc += all[((size_t)s * group + g) * rec + d] * wts[g * DECODE_MAX_SPLITS + s];
        emit(out, tc, ts, (size_t)h * group * HD + e, acc / gl[g]);
    }
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

#define DECODE_INST(HD, KIND) \
    template __global__ void attn_decode_kernel<HD, KIND>(DecodeArgs);
DECODE_INST(64, KV_F16)
DECODE_INST(128, KV_F16)
DECODE_INST(64, KV_F32)
DECODE_INST(128, KV_F32)
DECODE_INST(64, KV_Q8)
DECODE_INST(128, KV_Q8)

hipError_t launch_decode(int hd, int kind, const DecodeArgs& a, int kv_heads, int nseq, hipStream_t st) {
    dim3 grid(a.splits, kv_heads, nseq), block(DT);
#define L(HD, KIND) \
    if (hd == HD && kind == KIND) { hipLaunchKernelGGL((attn_decode_kernel<HD, KIND>), grid, block, 0, st, a); return hipGetLastError(); }
    L(64, KV_F16) L(128, KV_F16) L(64, KV_F32) L(128, KV_F32) L(64, KV_Q8) L(128, KV_Q8)
#undef L
    return hipErrorInvalidValue;
}

}  // namespace llmtie
