// Line order: a 64-key tile of the reference cache layouts (K [key][dim], V
// transposed [dim][key], f16) staged in LDS by direct-to-LDS loads that each
// read whole 128-byte lines, shared by the prefill and decode kernels.
//
// Gathered in MFMA fragment order instead, a wave-wide 16-byte-per-lane load
// touches 16 keys (or 16 V^T rows) in sixteen lines, half of each; where a
// launch keeps few waves per compute unit, the unit's rate of line requests
// then sets the time to a tile. In line order every instruction reads 1 KB =
// 8 whole lines:
//   K: instruction f (f < KF = HD / 8) holds tile keys f * KPI .. + KPI - 1
//      (a key is CR = HD / 8 chunks of 16 bytes, KPI = 64 / CR keys), lane l
//      chunk position l % CR of key f * KPI + l / CR;
//   V: instruction KF + f holds dims 8f .. 8f + 7, lane l position l % 8 of
//      dim 8f + l / 8 (a V^T row's 64 tile keys are one line).
// Within a key (dim) the chunk at position p is the row's chunk p ^ sw
// (pfl_ksw, pfl_vsw), chosen so that a fragment read, whose 16 lanes of a
// row take one chunk each of 16 keys (or 16 consecutive dims), lands on 16
// different 16-byte bank groups. pfl_kslot / pfl_vslot give a chunk's slot.
// The tile is the prefill's LDS tile: KF K slots of 1 KB, then KF V slots.
#pragma once
#include "common.h"

namespace llmtie {

template <int HD>
__device__ __forceinline__ int pfl_ksw(int k) {
    // hd 128 (a row is 16 chunks, 4 keys an instruction): the read's lanes
    // differ in k & 3 and (k >> 3) & 3; hd 64 (8 chunks, 8 keys): the slot's
    // bank group is 8 (k & 1) + position, so the swizzle takes (k >> 1) & 1
    // and (k >> 3) & 3.
    return HD == 128 ? ((k & 3) | (((k >> 3) & 3) << 2)) : (((k >> 1) & 1) | (((k >> 3) & 3) << 1));
}
__device__ __forceinline__ int pfl_vsw(int d) { return (d >> 1) & 7; }
// 16-byte slot of chunk c (dims 8c .. 8c + 7) of tile key k in the K area.
template <int HD>
__device__ __forceinline__ int pfl_kslot(int k, int c) {
    constexpr int CR = HD / 8, KPI = 64 / CR;
    return (k / KPI) * 64 + (k % KPI) * CR + (c ^ pfl_ksw<HD>(k));
}
// 16-byte slot of chunk c (tile keys 8c .. 8c + 7) of dim d in the V area.
__device__ __forceinline__ int pfl_vslot(int d, int c) { return (d >> 3) * 64 + (d & 7) * 8 + (c ^ pfl_vsw(d)); }
// One line-order load instruction of a reference-layout tile at kv0:
// fragment index f < KF is K, else V (see above).
template <int HD, int KF>
__device__ __forceinline__ void pfl_issue(const half_t* kc, __amdgpu_buffer_rsrc_t rv, int f, int lane, size_t kh,
                                          size_t cap, int kv0, int ktot, half_t* l) {
    constexpr int CR = HD / 8, KPI = 64 / CR;
    if (f < KF) {
        const int k = f * KPI + lane / CR;
        const int c = (lane % CR) ^ pfl_ksw<HD>(k);
        const int key = min(kv0 + k, ktot - 1);
        __builtin_amdgcn_global_load_lds(kc + (kh * cap + key) * HD + 8 * c, l, 16, 0, 0);
    } else {
        const int d = 8 * (f - KF) + (lane >> 3);
        const int c = (lane & 7) ^ pfl_vsw(d);
        const uint32_t off = (uint32_t)(((kh * HD + d) * cap + kv0 + 8 * c) * 2);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, l, 16, off, 0, 0, 0);
    }
}
// Zero the V entries of keys >= ktot in the tile at kv0 (line order when LO,
// else fragment order), threads tid, tid + nt, ... over the V area.
template <int HD, bool LO>
__device__ __forceinline__ void pf_zero_tail(half8* vf, int kv0, int ktot, int tid, int nt) {
    constexpr int NT = HD / 16, VF = 2 * NT;
    for (int c = tid; c < VF * 64; c += nt) {
        int k0;
        if constexpr (LO) {
            const int d = 8 * (c >> 6) + ((c & 63) >> 3);
            k0 = kv0 + 8 * ((c & 7) ^ pfl_vsw(d));
        } else {
            const int hf = c / (NT * 64), ln = c % 64;
            k0 = kv0 + 32 * hf + 8 * (ln >> 4);
        }
        if (k0 + 8 > ktot) {
            half8 x = vf[c];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (k0 + j >= ktot) x[j] = (half_t)0.0f;
            vf[c] = x;
        }
    }
}

}  // namespace llmtie
