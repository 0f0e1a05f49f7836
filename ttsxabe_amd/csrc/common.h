// Shared device helpers for the gfx950 attention kernels.
//
// Everything here is written for CDNA4 directly: 64-lane wavefronts, the
// v_mfma_f32_16x16x32_f16 matrix instruction, v_exp_f32 for exponentials and
// v_cvt_f16_f32 (round to nearest even) for every f32 -> f16 step.
//
// MFMA 16x16x32 f16 operand layout, as used by every kernel in this library
// (lane l of a 64-lane wave; `col = l & 15`, `grp = l >> 4`):
//   A (16 x 32):  lane l holds A[row = col][k = kslot(grp, j)], j = 0..7
//   B (32 x 16):  lane l holds B[k = kslot(grp, j)][col = col], j = 0..7
//   D (16 x 16):  lane l holds D[row = 4 * grp + r][col = col],  r = 0..3
// A and B name the same contraction slot for the same (grp, j), whatever the
// hardware's internal order of k is, so a kernel is free to decide which
// element of its own problem sits in slot (grp, j) as long as it decides it
// the same way for both operands. The kernels use that freedom to land the
// softmax probabilities straight in B-operand order without an LDS round trip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define LLMTIE_WAVE 64
#define LLMTIE_LOG2E 1.4426950408889634f

__device__ __forceinline__ floatx4 mfma16(half8 a, half8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 2^x on the transcendental unit; 2^-inf is exactly 0.
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float ninf() { return __builtin_bit_cast(float, 0xff800000u); }

// f32 -> f16, IEEE round to nearest even (v_cvt_f16_f32 in the default mode).
__device__ __forceinline__ half_t to_h(float x) { return (half_t)x; }

// x = hi + lo with hi = f16(x), lo = f16(x - hi): the pair carries ~22 bits
// of x, so an MFMA against both halves reproduces an f32 product to about
// 2^-22 relative instead of f16's 2^-11.
__device__ __forceinline__ void split_h(float x, half_t& hi, half_t& lo) {
    hi = (half_t)x;
    lo = (half_t)(x - (float)hi);
}

__device__ __forceinline__ half8 zero_h8() {
    half8 z;
#pragma unroll
    for (int j = 0; j < 8; ++j) z[j] = (half_t)0.0f;
    return z;
}

__device__ __forceinline__ floatx4 zero_f4() {
    floatx4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    return z;
}

// 16 bytes as eight halves; `p` must be 16-byte aligned.
__device__ __forceinline__ half8 ld_h8(const void* p) {
    return *reinterpret_cast<const half8*>(p);
}

// Eight halves from an address that is only 4-byte aligned.
__device__ __forceinline__ half8 ld_h8_a4(const uint16_t* p) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(p);
    uint32_t x0 = w[0], x1 = w[1], x2 = w[2], x3 = w[3];
    half8 r;
    uint32_t ws[4] = {x0, x1, x2, x3};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r[2 * i] = __builtin_bit_cast(half_t, (uint16_t)(ws[i] & 0xffffu));
        r[2 * i + 1] = __builtin_bit_cast(half_t, (uint16_t)(ws[i] >> 16));
    }
    return r;
}

// Eight int8 codes (8 bytes, 8-byte aligned) as eight exact halves.
__device__ __forceinline__ half8 ld_q8x8(const int8_t* p) {
    const uint2 w = *reinterpret_cast<const uint2*>(p);
    half8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r[i] = (half_t)(float)(int8_t)((w.x >> (8 * i)) & 0xff);
        r[4 + i] = (half_t)(float)(int8_t)((w.y >> (8 * i)) & 0xff);
    }
    return r;
}

// Cross-lane reductions over the four lanes that share `col` (xor 16, 32),
// on the VALU rather than through the LDS crossbar. v_permlane16_swap with
// both operands = v exchanges the odd 16-lane row of each row pair with the
// even one, so afterwards the two results hold, in every lane of the pair,
// the even row's v and the odd row's v; v_permlane32_swap does the same for
// the two 32-lane halves. Combining the two results is then the pairwise
// step of the reduction (commutative, so every lane gets identical bits).
__device__ __forceinline__ float max4grp(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum4grp(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Whole-wave max and sum, every lane getting the same bits, on the VALU:
// DPP xor-1 and xor-2 within quads, the half-row and row mirrors (lane i
// with 7 - i, then 15 - i), then the two permlane swaps across rows and
// halves. Each step combines a lane with a partner that combines it back,
// so partners compute identical values (no LDS-crossbar round trips).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xb1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f<0x4e>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_f<0x140>(v));  // row_mirror
    return max4grp(v);
}
__device__ __forceinline__ float wave_sum(float v) {
    v = v + dpp_f<0xb1>(v);
    v = v + dpp_f<0x4e>(v);
    v = v + dpp_f<0x141>(v);
    v = v + dpp_f<0x140>(v);
    return sum4grp(v);
}

// Agent-scope (device-coherent) 32-bit store and loads: visible across the
// XCDs' separate L2s without a cache-wide fence.
__device__ __forceinline__ void st_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wide reads of a workgroup-uniform region through a buffer resource: one
// 8- or 16-byte load per lane, reads past `bytes` return zeros (so a ragged
// tail needs no branch), and AUX is the cache policy: AUX_AGENT (sc1, the
// policy of an agent-scope relaxed atomic load) for data another workgroup
// of this launch published with st_coherent, AUX_XCD (sc0) for data another
// workgroup on the same XCD stored into the shared L2 in this launch, 0 for
// data an earlier launch wrote.
constexpr int AUX_AGENT = 16;
constexpr int AUX_XCD = 1;
// Data read once and never again in the launch (a decode's KV stream): sc0
// plus the non-temporal bit, so the stream does not displace what the L2
// and the Infinity Cache hold for reuse (C5: 66.6 -> 62.5 us).
constexpr int AUX_STREAM = 3;
struct Region {
    __amdgpu_buffer_rsrc_t r;
};
__device__ __forceinline__ Region region(const void* base, uint32_t bytes) {
    // Word 3 = 0x00020000: raw (untyped) buffer access on gfx9-family parts.
    return Region{__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000)};
}
template <int AUX>
__device__ __forceinline__ float4 ld_region4(const Region& g, uint32_t off) {
    typedef float v4 __attribute__((ext_vector_type(4)));
    const v4 x = __builtin_amdgcn_raw_buffer_load_b128(g.r, off, 0, AUX);
    return make_float4(x[0], x[1], x[2], x[3]);
}
template <int AUX>
__device__ __forceinline__ float2 ld_region2(const Region& g, uint32_t off) {
    typedef float v2 __attribute__((ext_vector_type(2)));
    const v2 x = __builtin_amdgcn_raw_buffer_load_b64(g.r, off, 0, AUX);
    return make_float2(x[0], x[1]);
}

// Calls f(std::integral_constant<int, i>{}) for i = 0 .. N-1, unrolled, so a
// loop index can select registers (an index chosen at run time would put a
// register array in scratch).
template <int... I, typename F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, I...>, F&& f) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(std::make_integer_sequence<int, N>{}, f);
}
