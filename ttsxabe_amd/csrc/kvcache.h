// Launch interface of the KV-cache producers (kvcache.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmtie {

hipError_t launch_rope(float* x, long off, const float* div, int t, int heads, int hd, float theta, int first,
                       hipStream_t st);
hipError_t launch_append(const float* src, long src_off, void* dst, int f16, int tr, int n, int kv, int hd, int cap,
                         int past, hipStream_t st);
hipError_t launch_rope_cache_f16(float* q, long q_off, const float* k, long k_off, const float* v, long v_off,
                                 const float* div, int heads, int kv, int hd, float theta, int pos, uint16_t* kc,
                                 uint16_t* vc, int cap, hipStream_t st);
hipError_t launch_grow(const void* src, void* dst, int esz, int rows, int len, int ss, int ds, hipStream_t st);
hipError_t launch_append_q8(const float* k, long k_off, const float* v, long v_off, char* cache, int slot, int n,
                            int kv, int hd, int cap, int past, hipStream_t st);
hipError_t launch_rope_cache_q8(float* q, long q_off, const float* k, long k_off, const float* v, long v_off,
                                const float* div, int heads, int kv, int hd, float theta, int pos, char* cache,
                                int slot, int cap, hipStream_t st);
hipError_t launch_append_t16(const float* src, long src_off, uint16_t* cache, int n, int kv, int hd, int cap,
                             int past, int value, hipStream_t st);
hipError_t launch_rope_cache_t16(float* q, long q_off, const float* k, long k_off, const float* v, long v_off,
                                 const float* div, int heads, int kv, int hd, float theta, int pos, uint16_t* cache,
                                 int cap, hipStream_t st);
hipError_t launch_ref_to_t16(const uint16_t* k, const uint16_t* v, uint16_t* cache, int kv, int hd, int cap, int live,
                             int tcap, hipStream_t st);

}  // namespace llmtie
