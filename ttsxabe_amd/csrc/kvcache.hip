// KV-cache producers: RoPE, append (f32 / f16 / Q8_0), fused rotate+append,
// and growth, all writing the layouts the attention kernels read.
//
// Replaces crates/llmtie-cuda/src/kernels.rs:4908-4948 (`rope`),
// :5244-5318 (`cache_append[_t][_f16]`), :5334-5380 (`rope_cache_f16`) and
// :5397-5423 (`cache_grow[_f16]`). The Q8_0 producers have no reference
// counterpart (the reference holds no quantized KV cache); they quantize as
// ggml's `quantize_row_q8_0_ref` does: d = max|x| / 127, code = round-half-
// away(x / d), d stored as f16, one block per 32 dims of one position.
//
// These are tiny launch-bound kernels: a flat index per element, coalesced
// over the source row, scattered into the destination layout.
#include "common.h"
#include "kvcache.h"
#include "kvlayout.h"

// No multiply-add contraction in this file: the rotations are the reference's
// separate f32 multiplies and subtraction, so the fused rotate+append and the
// separate rope then append produce the same bits whatever the kernel.
#pragma clang fp contract(off)

namespace llmtie {

constexpr int KB = 256;

// RoPE angle of pair j at position p, in f32 as the reference's CPU twin
// (crates/llmtie-dsp/src/rope.rs:83-126) computes it.
__device__ __forceinline__ void rope_sc(int j, int hd, float theta, const float* div, int p, float& sn, float& cs) {
    float inv = powf(theta, -2.0f * (float)j / (float)hd);
    if (div) inv /= div[j];
    sincosf((float)p * inv, &sn, &cs);
}

__global__ __launch_bounds__(KB) void rope_kernel(float* x, long off, const float* div, int t, int heads, int hd,
                                                  float theta, int first) {
    const int half = hd >> 1;
    const long i = (long)blockIdx.x * KB + threadIdx.x;
    if (i >= (long)t * heads * half) return;
    const int j = (int)(i % half);
    const int hh = (int)((i / half) % heads);
    const int p = (int)(i / ((long)half * heads));
    float sn, cs;
    rope_sc(j, hd, theta, div, first + p, sn, cs);
    const size_t b = (size_t)off + ((size_t)p * heads + hh) * hd + j;
    const float a0 = x[b], b0 = x[b + half];
    x[b] = a0 * cs - b0 * sn;
    x[b + half] = b0 * cs + a0 * sn;
}

// f32 or f16 append of n rows [n][kv*hd] into K [kv][cap][hd] or (transposed)
// V [kv][hd][cap] at positions past..past+n-1.
template <typename T, bool TR>
__global__ __launch_bounds__(KB) void append_kernel(const float* src, long src_off, T* dst, int n, int kv, int hd,
                                                    int cap, int past) {
    const long i = (long)blockIdx.x * KB + threadIdx.x;
    const int d = kv * hd;
    if (i >= (long)n * d) return;
    const int ti = (int)(i / d);
    const int hh = (int)((i % d) / hd);
    const int j = (int)(i % hd);
    const float x = src[src_off + i];
    const size_t at = TR ? ((size_t)hh * hd + j) * cap + past + ti : ((size_t)hh * cap + past + ti) * hd + j;
    if constexpr (sizeof(T) == 2) {
        dst[at] = __builtin_bit_cast(uint16_t, to_h(x));
    } else {
        dst[at] = x;
    }
}

// q rotated in place; k rotated and v copied into the f16 caches at `pos`.
__global__ __launch_bounds__(KB) void rope_cache_f16_kernel(float* q, long q_off, const float* k, long k_off,
                                                            const float* v, long v_off, const float* div,
                                                            int heads, int kv, int hd, float theta, int pos,
                                                            uint16_t* kc, uint16_t* vc, int cap) {
    const int half = hd >> 1;
    const int nq = heads * half, nk = kv * half, nv = kv * hd;
    const int i = blockIdx.x * KB + threadIdx.x;
    if (i < nq + nk) {
        const bool is_q = i < nq;
        const int e = is_q ? i : i - nq;
        const int j = e % half, hh = e / half;
        float sn, cs;
        rope_sc(j, hd, theta, div, pos, sn, cs);
        if (is_q) {
            const size_t b = (size_t)q_off + (size_t)hh * hd + j;
            const float a0 = q[b], b0 = q[b + half];
            q[b] = a0 * cs - b0 * sn;
            q[b + half] = b0 * cs + a0 * sn;
        } else {
            const size_t b = (size_t)k_off + (size_t)hh * hd + j;
            const float a0 = k[b], b0 = k[b + half];
            uint16_t* d = kc + ((size_t)hh * cap + pos) * hd;
            d[j] = __builtin_bit_cast(uint16_t, to_h(a0 * cs - b0 * sn));
            d[j + half] = __builtin_bit_cast(uint16_t, to_h(b0 * cs + a0 * sn));
        }
    } else if (i < nq + nk + nv) {
        const int e = i - nq - nk;
        const int hh = e / hd, j = e % hd;
        vc[((size_t)hh * hd + j) * cap + pos] = __builtin_bit_cast(uint16_t, to_h(v[(size_t)v_off + e]));
    }
}

template <typename T>
__global__ __launch_bounds__(KB) void grow_kernel(const T* src, T* dst, int rows, int len, int ss, int ds) {
    const long i = (long)blockIdx.x * KB + threadIdx.x;
    if (i >= (long)rows * len) return;
    const int r = (int)(i / len), j = (int)(i % len);
    dst[(size_t)r * ds + j] = src[(size_t)r * ss + j];
}

// One Q8_0 block per 32 consecutive threads: the 32 dims [32b, 32b+32) of
// one (position, kv head) row. `x` is this thread's element.
__device__ __forceinline__ void q8_block(float x, int8_t& code, uint16_t& dbits) {
    float amax = fabsf(x);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    code = (int8_t)(int)roundf(x * id);
    dbits = __builtin_bit_cast(uint16_t, to_h(d));
}

// Byte offsets of element (position p, dim d) of (slot, kv head) `kvh` in a
// tiled Q8_0 cache (kvlayout.h): codes and the scale of its dim block.
struct Q8At {
    long code, scale;
};
__device__ __forceinline__ Q8At q8_at(size_t kvh, int nblk, int hd, int p, int d, bool value) {
    const long blk = ((long)kvh * nblk + (p >> 5)) * tq8_block_bytes(hd);
    const int kk = p & 31;
    Q8At r;
    r.code = blk + (value ? 32L * hd + tq8_v_off(kk, d) : tq8_k_off(hd, kk, d));
    r.scale = blk + 64L * hd + (value ? 64L * (hd / 32) : 0) + 2L * ((d >> 5) * 32 + kk);
    return r;
}

// n rows [n][kv*hd] of K (already rotated) and V into slot `slot` of a tiled
// Q8_0 cache at positions past..past+n-1.
__global__ __launch_bounds__(KB) void append_q8_kernel(const float* k, long k_off, const float* v, long v_off,
                                                       char* cache, int slot, int n, int kv, int hd, int cap,
                                                       int past) {
    const long i = (long)blockIdx.x * KB + threadIdx.x;
    const int d = kv * hd;
    const long total = (long)n * d;
    // Threads past the end still take part in the block-wide shuffles as
    // zeros; total is a multiple of 32, so they are whole groups.
    const bool live = i < total;
    const long ii = live ? i : 0;
    const int ti = (int)(ii / d);
    const int hh = (int)((ii % d) / hd);
    const int j = (int)(ii % hd);
    const size_t kvh = (size_t)slot * kv + hh;
    const int nb = tiled_nblk(cap);
    int8_t c;
    uint16_t db;
    q8_block(live ? k[k_off + ii] : 0.0f, c, db);
    if (live) {
        const Q8At at = q8_at(kvh, nb, hd, past + ti, j, false);
        cache[at.code] = (char)(c ^ 0x80);
        if ((j & 31) == 0) *reinterpret_cast<uint16_t*>(cache + at.scale) = db;
    }
    q8_block(live ? v[v_off + ii] : 0.0f, c, db);
    if (live) {
        const Q8At at = q8_at(kvh, nb, hd, past + ti, j, true);
        cache[at.code] = (char)(c ^ 0x80);
        if ((j & 31) == 0) *reinterpret_cast<uint16_t*>(cache + at.scale) = db;
    }
}

// The Q8_0 twin of rope_cache_f16: q rotated in place, k rotated and
// quantized, v quantized, into slot `slot` at position `pos`. Thread e owns
// output element e of the rotated k row (or, past nk, of v), so a block of
// 32 consecutive threads is one Q8_0 block.
__global__ __launch_bounds__(KB) void rope_cache_q8_kernel(float* q, long q_off, const float* k, long k_off,
                                                           const float* v, long v_off, const float* div,
                                                           int heads, int kv, int hd, float theta, int pos,
                                                           char* cache, int slot, int cap) {
    const int half = hd >> 1;
    const int nq = heads * half;  // q pairs
    const int nk = kv * hd;       // rotated k elements
    const int nv = kv * hd;
    // Blocks [0, qb) rotate q; the rest quantize k then v. Keeping the two
    // phases in different blocks keeps each k/v block of 32 threads whole.
    const int qblocks = (nq + KB - 1) / KB;
    if ((int)blockIdx.x < qblocks) {
        const int i = blockIdx.x * KB + threadIdx.x;
        if (i >= nq) return;
        const int j = i % half, hh = i / half;
        float sn, cs;
        rope_sc(j, hd, theta, div, pos, sn, cs);
        const size_t b = (size_t)q_off + (size_t)hh * hd + j;
        const float a0 = q[b], b0 = q[b + half];
        q[b] = a0 * cs - b0 * sn;
        q[b + half] = b0 * cs + a0 * sn;
        return;
    }
    const int i = (blockIdx.x - qblocks) * KB + threadIdx.x;
    const bool live = i < nk + nv;
    const bool is_k = i < nk;
    const int e = live ? (is_k ? i : i - nk) : 0;
    const int hh = e / hd, jj = e % hd;
    float x = 0.0f;
    if (live && is_k) {
        const int j = jj % half;
        float sn, cs;
        rope_sc(j, hd, theta, div, pos, sn, cs);
        const size_t b = (size_t)k_off + (size_t)hh * hd + j;
        const float a0 = k[b], b0 = k[b + half];
        x = jj < half ? a0 * cs - b0 * sn : b0 * cs + a0 * sn;
    } else if (live) {
        x = v[(size_t)v_off + e];
    }
    int8_t c;
    uint16_t db;
    q8_block(x, c, db);
    if (!live) return;
    const Q8At at = q8_at((size_t)slot * kv + hh, tiled_nblk(cap), hd, pos, jj, !is_k);
    cache[at.code] = (char)(c ^ 0x80);
    if ((jj & 31) == 0) *reinterpret_cast<uint16_t*>(cache + at.scale) = db;
}

// ------------------------------------------------------------ tiled f16

// Half offset of element (position p, dim d) of kv head h in a tiled f16 cache.
__device__ __forceinline__ long t16_at(int h, int nblk, int hd, int p, int d, bool value) {
    const long blk = ((long)h * nblk + (p >> 5)) * 64L * hd;
    return blk + (value ? 32L * hd + t16_v_off(p & 31, d) : t16_k_off(hd, p & 31, d));
}

// The tiled twin of cache_append_f16: n rows [n][kv*hd] into positions
// past.. of the K (or, `value`, the V) area.
__global__ __launch_bounds__(KB) void append_t16_kernel(const float* src, long src_off, uint16_t* cache, int n,
                                                        int kv, int hd, int cap, int past, int value) {
    const long i = (long)blockIdx.x * KB + threadIdx.x;
    const int d = kv * hd;
    if (i >= (long)n * d) return;
    const int ti = (int)(i / d);
    const int hh = (int)((i % d) / hd);
    const int j = (int)(i % hd);
    cache[t16_at(hh, tiled_nblk(cap), hd, past + ti, j, value)] =
        __builtin_bit_cast(uint16_t, to_h(src[src_off + i]));
}

// The tiled twin of rope_cache_f16.
__global__ __launch_bounds__(KB) void rope_cache_t16_kernel(float* q, long q_off, const float* k, long k_off,
                                                            const float* v, long v_off, const float* div,
                                                            int heads, int kv, int hd, float theta, int pos,
                                                            uint16_t* cache, int cap) {
    const int half = hd >> 1;
    const int nq = heads * half, nk = kv * half, nv = kv * hd;
    const int nb = tiled_nblk(cap);
    const int i = blockIdx.x * KB + threadIdx.x;
    if (i < nq + nk) {
        const bool is_q = i < nq;
        const int e = is_q ? i : i - nq;
        const int j = e % half, hh = e / half;
        float sn, cs;
        rope_sc(j, hd, theta, div, pos, sn, cs);
        if (is_q) {
            const size_t b = (size_t)q_off + (size_t)hh * hd + j;
            const float a0 = q[b], b0 = q[b + half];
            q[b] = a0 * cs - b0 * sn;
            q[b + half] = b0 * cs + a0 * sn;
        } else {
            const size_t b = (size_t)k_off + (size_t)hh * hd + j;
            const float a0 = k[b], b0 = k[b + half];
            cache[t16_at(hh, nb, hd, pos, j, false)] = __builtin_bit_cast(uint16_t, to_h(a0 * cs - b0 * sn));
            cache[t16_at(hh, nb, hd, pos, j + half, false)] = __builtin_bit_cast(uint16_t, to_h(b0 * cs + a0 * sn));
        }
    } else if (i < nq + nk + nv) {
        const int e = i - nq - nk;
        const int hh = e / hd, j = e % hd;
        cache[t16_at(hh, nb, hd, pos, j, true)] = __builtin_bit_cast(uint16_t, to_h(v[(size_t)v_off + e]));
    }
}

// Reference-layout f16 caches (K [kv][cap][hd], V [kv][hd][cap]) into the
// tiled layout, positions 0..live-1 (the rest of the last block is zeroed).
__global__ __launch_bounds__(KB) void ref_to_t16_kernel(const uint16_t* k, const uint16_t* v, uint16_t* cache, int kv,
                                                        int hd, int cap, int live, int tcap) {
    const long i = (long)blockIdx.x * KB + threadIdx.x;
    const int nbl = (live + 31) / 32;
    const long per = (long)nbl * 32 * hd;  // elements per head and area
    if (i >= 2L * kv * per) return;
    const bool value = i >= (long)kv * per;
    const long e = value ? i - (long)kv * per : i;
    const int hh = (int)(e / per);
    const int p = (int)((e % per) / hd), d = (int)(e % hd);
    uint16_t x = 0;
    if (p < live) x = value ? v[((size_t)hh * hd + d) * cap + p] : k[((size_t)hh * cap + p) * hd + d];
    cache[t16_at(hh, tiled_nblk(tcap), hd, p, d, value)] = x;
}

static inline unsigned nblk(long n) { return (unsigned)((n + KB - 1) / KB); }

hipError_t launch_rope(float* x, long off, const float* div, int t, int heads, int hd, float theta, int first,
                       hipStream_t st) {
    const long n = (long)t * heads * (hd / 2);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_kernel, dim3(nblk(n)), dim3(KB), 0, st, x, off, div, t, heads, hd, theta, first);
    return hipGetLastError();
}

hipError_t launch_append(const float* src, long src_off, void* dst, int f16, int tr, int n, int kv, int hd, int cap,
                         int past, hipStream_t st) {
    const long tot = (long)n * kv * hd;
    if (tot == 0) return hipSuccess;
    dim3 g(nblk(tot)), b(KB);
    if (f16) {
        if (tr) hipLaunchKernelGGL((append_kernel<uint16_t, true>), g, b, 0, st, src, src_off, (uint16_t*)dst, n, kv, hd, cap, past);
        else hipLaunchKernelGGL((append_kernel<uint16_t, false>), g, b, 0, st, src, src_off, (uint16_t*)dst, n, kv, hd, cap, past);
    } else {
        if (tr) hipLaunchKernelGGL((append_kernel<float, true>), g, b, 0, st, src, src_off, (float*)dst, n, kv, hd, cap, past);
        else hipLaunchKernelGGL((append_kernel<float, false>), g, b, 0, st, src, src_off, (float*)dst, n, kv, hd, cap, past);
    }
    return hipGetLastError();
}

hipError_t launch_rope_cache_f16(float* q, long q_off, const float* k, long k_off, const float* v, long v_off,
                                 const float* div, int heads, int kv, int hd, float theta, int pos, uint16_t* kc,
                                 uint16_t* vc, int cap, hipStream_t st) {
    const long n = (long)heads * (hd / 2) + (long)kv * (hd / 2) + (long)kv * hd;
    hipLaunchKernelGGL(rope_cache_f16_kernel, dim3(nblk(n)), dim3(KB), 0, st, q, q_off, k, k_off, v, v_off, div,
                       heads, kv, hd, theta, pos, kc, vc, cap);
    return hipGetLastError();
}

hipError_t launch_grow(const void* src, void* dst, int esz, int rows, int len, int ss, int ds, hipStream_t st) {
    const long n = (long)rows * len;
    if (n == 0) return hipSuccess;
    if (esz == 2) hipLaunchKernelGGL((grow_kernel<uint16_t>), dim3(nblk(n)), dim3(KB), 0, st, (const uint16_t*)src, (uint16_t*)dst, rows, len, ss, ds);
    else if (esz == 1) hipLaunchKernelGGL((grow_kernel<int8_t>), dim3(nblk(n)), dim3(KB), 0, st, (const int8_t*)src, (int8_t*)dst, rows, len, ss, ds);
    else hipLaunchKernelGGL((grow_kernel<float>), dim3(nblk(n)), dim3(KB), 0, st, (const float*)src, (float*)dst, rows, len, ss, ds);
    return hipGetLastError();
}

hipError_t launch_append_q8(const float* k, long k_off, const float* v, long v_off, char* cache, int slot, int n,
                            int kv, int hd, int cap, int past, hipStream_t st) {
    const long tot = (long)n * kv * hd;
    if (tot == 0) return hipSuccess;
    hipLaunchKernelGGL(append_q8_kernel, dim3(nblk(tot)), dim3(KB), 0, st, k, k_off, v, v_off, cache, slot, n, kv, hd,
                       cap, past);
    return hipGetLastError();
}

hipError_t launch_rope_cache_q8(float* q, long q_off, const float* k, long k_off, const float* v, long v_off,
                                const float* div, int heads, int kv, int hd, float theta, int pos, char* cache,
                                int slot, int cap, hipStream_t st) {
    const unsigned qb = nblk((long)heads * (hd / 2));
    const unsigned kb = nblk(2L * kv * hd);
    hipLaunchKernelGGL(rope_cache_q8_kernel, dim3(qb + kb), dim3(KB), 0, st, q, q_off, k, k_off, v, v_off, div,
                       heads, kv, hd, theta, pos, cache, slot, cap);
    return hipGetLastError();
}

hipError_t launch_append_t16(const float* src, long src_off, uint16_t* cache, int n, int kv, int hd, int cap,
                             int past, int value, hipStream_t st) {
    const long tot = (long)n * kv * hd;
    if (tot == 0) return hipSuccess;
    hipLaunchKernelGGL(append_t16_kernel, dim3(nblk(tot)), dim3(KB), 0, st, src, src_off, cache, n, kv, hd, cap,
                       past, value);
    return hipGetLastError();
}

hipError_t launch_rope_cache_t16(float* q, long q_off, const float* k, long k_off, const float* v, long v_off,
                                 const float* div, int heads, int kv, int hd, float theta, int pos, uint16_t* cache,
                                 int cap, hipStream_t st) {
    const long n = (long)heads * (hd / 2) + (long)kv * (hd / 2) + (long)kv * hd;
    hipLaunchKernelGGL(rope_cache_t16_kernel, dim3(nblk(n)), dim3(KB), 0, st, q, q_off, k, k_off, v, v_off, div,
                       heads, kv, hd, theta, pos, cache, cap);
    return hipGetLastError();
}

hipError_t launch_ref_to_t16(const uint16_t* k, const uint16_t* v, uint16_t* cache, int kv, int hd, int cap, int live,
                             int tcap, hipStream_t st) {
    const long n = 2L * kv * ((live + 31) / 32) * 32 * hd;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(ref_to_t16_kernel, dim3(nblk(n)), dim3(KB), 0, st, k, v, cache, kv, hd, cap, live, tcap);
    return hipGetLastError();
}

}  // namespace llmtie
