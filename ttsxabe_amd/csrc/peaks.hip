// Measurement probes (not part of the attention ABI): what this part sustains
// for the two resources the kernels are bound by, measured in the bench run
// itself. Built as a separate library, libllmtie_peaks.so.
//
//   llmtie_peak_mfma: back-to-back v_mfma_f32_16x16x32_f16 from registers, two
//     waves per SIMD with eight independent accumulators each (no memory
//     traffic): the MFMA rate at the clock the part holds under dense work.
//   llmtie_peak_read: a grid-stride 16-byte-per-lane read of a buffer larger
//     than the last-level cache: the HBM read rate a streaming kernel can
//     reach.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(512) void peak_mfma_kernel(float* sink, int iters) {
    const int t = threadIdx.x;
    half8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (_Float16)(0.001f * (float)((t + i) & 7));
        b[i] = (_Float16)(0.002f * (float)((t * 3 + i) & 7));
    }
    floatx4 c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c[j], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += c[j][0] + c[j][1] + c[j][2] + c[j][3];
    if (s == -1.0f) sink[blockIdx.x] = s;  // never true; keeps the chains live
}

__global__ __launch_bounds__(256) void peak_read_kernel(const uint4* __restrict__ p, size_t n, unsigned* sink) {
    uint4 acc = {0u, 0u, 0u, 0u};
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint4 v = p[i];
        acc.x ^= v.x;
        acc.y ^= v.y;
        acc.z ^= v.z;
        acc.w ^= v.w;
    }
    if ((acc.x & acc.y & acc.z & acc.w) == 0x9e3779b9u) sink[0] = acc.x;  // keeps the loads live
}

extern "C" {

// FLOPs issued: blocks * 8 waves * iters * 8 MFMAs * 16384.
int llmtie_peak_mfma(void* stream, float* sink, int blocks, int iters) {
    hipLaunchKernelGGL(peak_mfma_kernel, dim3(blocks), dim3(512), 0, static_cast<hipStream_t>(stream), sink, iters);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// Reads `bytes` (a multiple of 16) from `src`.
int llmtie_peak_read(void* stream, const void* src, size_t bytes, unsigned* sink, int blocks) {
    hipLaunchKernelGGL(peak_read_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4*>(src), bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // extern "C"
