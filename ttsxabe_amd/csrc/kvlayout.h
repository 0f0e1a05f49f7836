// The tiled KV-cache layouts ("fragment order"), shared by the producers
// (kvcache.hip), the decode kernel and the prefill kernel.
//
// A cache is cut into blocks of 32 positions. Inside a block the elements sit
// in exactly the order the 64 lanes of a wave consume them as
// v_mfma_f32_16x16x32_f16 operands, so every load of a block is one
// contiguous 1 KB wave-wide read (16 bytes per lane, consecutive lanes at
// consecutive addresses) and every LDS read of a staged block is
// conflict-free. Lane l = col + 16 * g (col = l & 15, g = l >> 4).
//
// f16 tiled block, head_dim HD (NS = HD/32 contraction steps, NT = HD/16 tiles):
//   K area, 32*HD halves: ((T*NS + s)*64 + l)*8 + j  holds
//       key 8*(col/4) + 4T + col%4, dim 32s + 8g + j        (T = 0, 1)
//   V area, 32*HD halves: (t*64 + l)*8 + j  holds  dim 16t + col, key 8g + j
//   A head's blocks are contiguous: block b of kv head h at (h*nblk + b) * 64*HD halves.
//
// Q8_0 tiled block (GGUF Q8_0: 32 int8 codes share one f16 scale d, value
// d * code; the 32 codes of a scale are 32 consecutive dims of one position).
// Codes are stored offset-binary (code + 128 as an unsigned byte, i.e. the
// sign bit flipped), the form the kernel splices straight into f16 bits:
//   K codes, 32*HD bytes: ((T*(NS/2) + s/2)*64 + l)*16 + 8*(s%2) + j  holds
//       key 8*(col/4) + 4T + col%4, dim 32s + 8g + j
//   V codes, 32*HD bytes: ((t/2)*64 + l)*16 + 8*(t%2) + j  holds  dim 16t + col, key 8g + j
//   K scales, 32*(HD/32) halves: [dim block][key]
//   V scales, the same (so the scales of 8 consecutive keys for one dim block
//   are one 16-byte read, and pair up with packed f16 probabilities).
//   Block bytes: 2*32*HD + 2*32*(HD/32)*2 (8704 at HD 128 = 272 per position).
//   Block b of (slot, kv head h) at ((slot*kv + h)*nblk + b) * block bytes.
#pragma once
#include <stdint.h>

namespace llmtie {

constexpr int KB_POS = 32;  // positions per tiled block

__host__ __device__ inline int tiled_nblk(int cap) { return (cap + KB_POS - 1) / KB_POS; }

// Offset (in halves, from the block's K area) of key kk, dim d.
__host__ __device__ inline int t16_k_off(int hd, int kk, int d) {
    const int ns = hd / 32;
    const int T = (kk >> 2) & 1, m = 4 * (kk >> 3) + (kk & 3);
    const int s = d >> 5, g = (d >> 3) & 3, j = d & 7;
    return ((T * ns + s) * 64 + (m + 16 * g)) * 8 + j;
}
// Offset (in halves, from the block's V area) of key kk, dim d.
__host__ __device__ inline int t16_v_off(int kk, int d) {
    const int t = d >> 4, c = d & 15, g = kk >> 3, j = kk & 7;
    return (t * 64 + (c + 16 * g)) * 8 + j;
}
// Offset (in bytes, from the block's K-code area) of key kk, dim d.
__host__ __device__ inline int tq8_k_off(int hd, int kk, int d) {
    const int ns = hd / 32;
    const int T = (kk >> 2) & 1, m = 4 * (kk >> 3) + (kk & 3);
    const int s = d >> 5, g = (d >> 3) & 3, j = d & 7;
    return ((T * (ns / 2) + (s >> 1)) * 64 + (m + 16 * g)) * 16 + 8 * (s & 1) + j;
}
// Offset (in bytes, from the block's V-code area) of key kk, dim d.
__host__ __device__ inline int tq8_v_off(int kk, int d) {
    const int t = d >> 4, c = d & 15, g = kk >> 3, j = kk & 7;
    return ((t >> 1) * 64 + (c + 16 * g)) * 16 + 8 * (t & 1) + j;
}
__host__ __device__ constexpr long tq8_block_bytes(int hd) { return 2L * 32 * hd + 2L * 32 * (hd / 32) * 2; }

}  // namespace llmtie
