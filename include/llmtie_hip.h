/*
 * llmtie_hip.h - C ABI of the MI355X (gfx950) fused-attention library.
 *
 * A drop-in replacement for the attention operators of the reference's
 * `llmtie_cuda::Gpu` (crates/llmtie-cuda/src/device.rs) and for the KV-cache
 * producers they read from. Every entry point takes plain device pointers with
 * element counts (so every bounds check the reference makes can still be made),
 * a hipStream_t passed as `void*` (NULL = the default stream), and returns a
 * status code named after the reference's `CudaError` variant
 * (crates/llmtie-cuda/src/error.rs:148-282). Shapes are refused before any
 * launch; a refused call touches no memory. Outputs are caller-owned.
 *
 * Calls are asynchronous on `stream` exactly like the reference's (one stream
 * per Gpu, device.rs:740-755). A decode scratch must not be shared by calls
 * that can run concurrently (device.rs:166-180).
 *
 * Layouts (as in the reference unless noted):
 *   q           [rows, heads * head_dim] f32, the heads of one GQA group adjacent
 *   K cache     [kv_heads, cap, head_dim]   (f32 or f16 bits)
 *   V cache     [kv_heads, head_dim, cap]   (transposed, f32 or f16 bits)
 *   tiled f16   (new) one buffer per layer, [kv_heads][blocks of 32 positions],
 *               each block K then V in MFMA fragment order (kvlayout.h)
 *   Q8_0 cache  (new; no reference counterpart) for `slots` sequences, tiled the
 *               same way: [slots][kv_heads][blocks], each block K codes, V
 *               codes, K scales, V scales; element = f16 scale * int8 code, one
 *               scale per 32 dims of one position (the GGUF Q8_0 block,
 *               crates/llmtie-gguf/src/dequant.rs:180-185); 272 bytes per
 *               position and kv head at head_dim 128.
 *   int8 twin   `n` int8 codes then `n / 32` f32 scales in one buffer (the
 *               reference's `Q8` buffer, device.rs:498-520)
 */
#ifndef LLMTIE_HIP_H
#define LLMTIE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: one per `CudaError` variant the attention path can raise. */
typedef enum llmtie_status {
    LLMTIE_OK = 0,
    LLMTIE_UNSUPPORTED_ATTENTION = 1, /* UnsupportedAttention{head_dim, heads, kv_heads} error.rs:270 */
    LLMTIE_ODD_CACHE_CAPACITY = 2,    /* OddCacheCapacity{cap}            error.rs:178 */
    LLMTIE_CACHE_OVERRUN = 3,         /* CacheOverrun{at, cap}            error.rs:162 */
    LLMTIE_SLICE_OVERRUN = 4,         /* SliceOverrun{at, len}            error.rs:149 */
    LLMTIE_RAGGED_BLOCK = 5,          /* RaggedBlock{k, block}            error.rs:63 */
    LLMTIE_MISMATCHED_Q8 = 6,         /* MismatchedQ8{rows, k, want_rows, want_k} error.rs:129 */
    LLMTIE_ODD_HEAD_DIM = 7,          /* OddHeadDim{head_dim}             error.rs:210 */
    LLMTIE_DRIVER = 8,                /* Driver{what, source}             error.rs:281 */
    LLMTIE_NO_DEVICE = 9,             /* NoDevice(String)                 error.rs:242 */
    LLMTIE_INVALID_ARGUMENT = 10,     /* a null pointer where a buffer is required (no reference twin) */
    LLMTIE_SCRATCH_GROWTH_IN_CAPTURE = 11, /* a decode scratch would have to grow while its stream captures a
                                            * graph (no reference twin: the reference does not capture);
                                            * fields: partial floats needed, held, counters needed, held */
    LLMTIE_SCRATCH_LIMIT = 12,             /* the fixed scratch of llmtie_attn_decode_f16_noalloc is too small
                                            * for the call (no reference twin); fields as above */
    LLMTIE_SPLIT_HEAD_LOST = 13            /* an earlier decode through this scratch wrote NaN for a head whose
                                            * split workgroups did not share an XCD (no reference twin; see
                                            * llmtie_decode_scratch_status); no fields */
} llmtie_status;

/* The last error raised on the calling thread: the status, up to four numeric
 * fields of the variant in its declaration order, and a rendered message. */
typedef struct llmtie_error {
    int status;
    size_t field[4];
    char message[240];
} llmtie_error;

/* Copies the calling thread's last error into *out; returns its status. */
int llmtie_last_error(llmtie_error* out);

/* Library version, "major.minor.patch". */
const char* llmtie_version(void);

/* Opaque decode scratch: split partials and arrival counters, grown on demand
 * and owned by the caller. Replaces `DecodeScratch::new()` (device.rs:219).
 * Its counters start at zero and every call leaves them at zero.
 * Graphs: a call captured into a HIP graph records the scratch's buffers.
 * Growth never frees a buffer: every replaced one stays allocated until
 * llmtie_decode_scratch_free, so an earlier graph keeps replaying correctly.
 * Growth is refused while the stream is capturing
 * (LLMTIE_SCRATCH_GROWTH_IN_CAPTURE): make one eager call of the largest shape
 * first. Freeing the scratch invalidates every graph that used it. */
typedef struct llmtie_decode_scratch llmtie_decode_scratch;
llmtie_decode_scratch* llmtie_decode_scratch_new(void);
void llmtie_decode_scratch_free(llmtie_decode_scratch* s);

/* The XCD-local split hand-off (no reference twin). When every XCD's run of a
 * launch's workgroups holds whole heads, a head's split partials pass
 * through that XCD's L2 instead of memory. The kernel checks that each head's
 * workgroups really shared an XCD; a head whose did not is written as NaN
 * (its int8 twin with NaN scales), never as a silently wrong context, and the
 * scratch records it in a host-visible word. The next decode call through the
 * scratch then returns LLMTIE_SPLIT_HEAD_LOST without launching, and
 * llmtie_decode_scratch_status returns (and clears) the same status after a
 * stream synchronisation; LLMTIE_OK otherwise. No failure has been seen on
 * gfx950, whose dispatcher deals workgroups L and L + 8k to one XCD; the
 * environment variable LLMTIE_DECODE_XCD=0 selects the coherent hand-off
 * everywhere (about 2 % slower at C2). The no-allocation entry point always
 * uses the coherent hand-off. */
int llmtie_decode_scratch_status(llmtie_decode_scratch* s);

/* Test hook (no reference twin; never needed in use): nonzero makes every
 * later decode report fake XCC ids (workgroup L as (L / 8) % 8) to the
 * XCD-local check, so a test can drive the check's failure path. */
void llmtie_debug_fake_xcc(int on);

/* ---------------------------------------------------------------- prefill */

/* Gpu::supports_flash (device.rs:5697): head_dim 64 or 128, heads a multiple
 * of kv_heads. */
int llmtie_supports_flash(size_t head_dim, size_t heads, size_t kv_heads);

/* Gpu::flash_attn (device.rs:5702): causal or full attention of tq query rows
 * (positions past .. past+tq-1) against an f32 cache holding past+tq keys.
 * out = [tq, heads*head_dim] f32.
 * The kernel rounds the f32 keys and values to f16 on their way into its
 * LDS tiles (the reference's arithmetic); nothing is allocated. */
int llmtie_flash_attn(void* stream, const float* q, size_t q_len, const float* k, size_t k_len,
                      const float* v, size_t v_len, float* out, size_t out_len, size_t tq, size_t past,
                      size_t heads, size_t kv_heads, size_t head_dim, size_t cap, float scale, int causal);

/* Gpu::flash_attn_f16 (device.rs:5754): the same against an f16 cache (cap even). */
int llmtie_flash_attn_f16(void* stream, const float* q, size_t q_len, const uint16_t* k, size_t k_len,
                          const uint16_t* v, size_t v_len, float* out, size_t out_len, size_t tq, size_t past,
                          size_t heads, size_t kv_heads, size_t head_dim, size_t cap, float scale, int causal);

/* Gpu::flash_attn_rows (device.rs:5812): non-causal attention over a stacked
 * [t, 3*heads*head_dim] q/k/v product, scale on q, context as f16 bits
 * [t, heads*head_dim]. head_dim 64. The rows are read where they lie and
 * rounded to f16 inside the kernel; nothing is allocated. */
int llmtie_flash_attn_rows(void* stream, const float* qkv, size_t qkv_len, uint16_t* out, size_t out_len,
                           size_t t, size_t heads, size_t head_dim, float scale);

/* ----------------------------------------------------------------- decode */

/* Gpu::attn_decode_f16 (device.rs:5949): one query row [heads*head_dim] over
 * tk live positions of an f16 cache; scale on q (scale_q) or on the scores.
 * Every decode entry accepts head_dim 64 and 128 and GQA groups up to 16: a
 * superset of the reference's refusals (it refuses groups over 4, 8 for its
 * head_dim-64 g8 kernel, device.rs:6245-6251, and an f32 cache at head_dim
 * 128, device.rs:6146). A binding that relies on those refusals to choose a
 * fallback refuses such shapes itself. */
int llmtie_attn_decode_f16(void* stream, const float* q, size_t q_len, const uint16_t* k, size_t k_len,
                           const uint16_t* v, size_t v_len, size_t heads, size_t kv_heads, size_t head_dim,
                           size_t tk, size_t cap, float scale, int scale_q, llmtie_decode_scratch* scratch,
                           float* out, size_t out_len);

/* No counterpart in the reference: llmtie_attn_decode_f16 for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments and result bits, no
 * scratch argument: the split partials and arrival counters live in a fixed
 * 4.25 MiB device array the library holds on each device (1M partial floats,
 * 256 kv heads' counters); a call that needs more is refused with
 * LLMTIE_SCRATCH_LIMIT before any launch. It calls no allocator. Every call
 * on one device shares that array, so calls that can overlap on one GPU (two
 * streams, two threads) race and must not be made. */
int llmtie_attn_decode_f16_noalloc(void* stream, const float* q, size_t q_len, const uint16_t* k, size_t k_len,
                                   const uint16_t* v, size_t v_len, size_t heads, size_t kv_heads, size_t head_dim,
                                   size_t tk, size_t cap, float scale, int scale_q, float* out, size_t out_len);

/* Gpu::attn_decode_f16_q (device.rs:5973): plus the context's int8 twin
 * (twin_len >= n + 4*(n/32) bytes, n = heads*head_dim). */
int llmtie_attn_decode_f16_q(void* stream, const float* q, size_t q_len, const uint16_t* k, size_t k_len,
                             const uint16_t* v, size_t v_len, size_t heads, size_t kv_heads, size_t head_dim,
                             size_t tk, size_t cap, float scale, int scale_q, llmtie_decode_scratch* scratch,
                             float* out, size_t out_len, int8_t* twin, size_t twin_len);

/* Gpu::attn_decode_f16_q_row (device.rs:6001): query from element q_off of q;
 * context into row `row` of out [rows, n] and of the twin [twin_rows, twin_k]. */
int llmtie_attn_decode_f16_q_row(void* stream, const float* q, size_t q_len, size_t q_off, const uint16_t* k,
                                 size_t k_len, const uint16_t* v, size_t v_len, size_t heads, size_t kv_heads,
                                 size_t head_dim, size_t tk, size_t cap, float scale, int scale_q,
                                 llmtie_decode_scratch* scratch, float* out, size_t out_len, int8_t* twin,
                                 size_t twin_rows, size_t twin_k, size_t row);

/* Gpu::attn_decode (device.rs:6132): the same off an f32 cache (head_dim 128
 * accepted as well as the reference's 64). */
int llmtie_attn_decode(void* stream, const float* q, size_t q_len, const float* k, size_t k_len, const float* v,
                       size_t v_len, size_t heads, size_t kv_heads, size_t head_dim, size_t tk, size_t cap,
                       float scale, int scale_q, llmtie_decode_scratch* scratch, float* out, size_t out_len);

/* Batched decode over a tiled GGUF Q8_0 cache (new; the reference's nearest
 * caller is Translator::step_rows, crates/llmtie-translate/src/model.rs:764,
 * which launches one f16 decode per row). nseq sequences in one launch:
 * sequence s attends its tk_dev[s] live positions of cache slot slot_dev[s];
 * q and out are [nseq, heads*head_dim]. tk_dev and slot_dev are device int32
 * arrays; max_tk bounds every tk_dev[s] (the kernel clamps to it, never
 * reading past it) and must be <= cap. A sequence whose slot is out of range
 * or whose length is 0 gets a NaN row. cache_len is in bytes
 * (llmtie_q8_cache_bytes). */
int llmtie_attn_decode_q8_batch(void* stream, const float* q, size_t q_len, const int8_t* cache, size_t cache_len,
                                size_t slots, const int32_t* tk_dev, const int32_t* slot_dev, size_t nseq,
                                size_t max_tk, size_t heads, size_t kv_heads, size_t head_dim, size_t cap,
                                float scale, int scale_q, llmtie_decode_scratch* scratch, float* out,
                                size_t out_len);

/* ------------------------------------------- tiled f16 cache (new layout)
 *
 * One buffer per layer holds K and V in fragment order, 32 positions a block
 * (see ttsxabe_amd/csrc/kvlayout.h): every load the decode and prefill kernels
 * make of it is a contiguous 1 KB wave-wide read. These mirror the reference
 * operators they are named after, with the two cache slices replaced by the
 * one tiled buffer; cap may be any positive count (rounded up to whole blocks
 * internally). */

/* Halves a tiled f16 cache of this shape holds. */
size_t llmtie_t16_cache_len(size_t kv_heads, size_t head_dim, size_t cap);

/* cache_append_f16 (device.rs:2849) into the tiled cache; value selects V. */
int llmtie_t16_append(void* stream, const float* src, size_t src_len, size_t src_off, uint16_t* cache,
                      size_t cache_len, size_t n, size_t kv_heads, size_t head_dim, size_t cap, size_t past,
                      int value);

/* rope_cache_f16 (device.rs:2915) into the tiled cache. */
int llmtie_t16_rope_cache(void* stream, float* q, size_t q_len, size_t q_off, const float* k, size_t k_len,
                          size_t k_off, const float* v, size_t v_len, size_t v_off, const float* freq_div,
                          size_t heads, size_t kv_heads, size_t head_dim, float theta, size_t pos, uint16_t* cache,
                          size_t cache_len, size_t cap);

/* cache_grow_f16 (device.rs:3152) for the tiled cache. */
int llmtie_t16_grow(void* stream, const uint16_t* src, size_t src_len, uint16_t* dst, size_t dst_len,
                    size_t kv_heads, size_t head_dim, size_t cap, size_t new_cap, size_t live);

/* Repack reference-layout f16 caches (positions 0..live-1) into a tiled one. */
int llmtie_t16_from_ref(void* stream, const uint16_t* k, size_t k_len, const uint16_t* v, size_t v_len,
                        size_t kv_heads, size_t head_dim, size_t cap, size_t live, uint16_t* cache,
                        size_t cache_len);

/* attn_decode_f16 (device.rs:5949) off the tiled cache. */
int llmtie_attn_decode_t16(void* stream, const float* q, size_t q_len, const uint16_t* cache, size_t cache_len,
                           size_t heads, size_t kv_heads, size_t head_dim, size_t tk, size_t cap, float scale,
                           int scale_q, llmtie_decode_scratch* scratch, float* out, size_t out_len);

/* attn_decode_f16_q_row (device.rs:6001) off the tiled cache; twin may be NULL. */
int llmtie_attn_decode_t16_q_row(void* stream, const float* q, size_t q_len, size_t q_off, const uint16_t* cache,
                                 size_t cache_len, size_t heads, size_t kv_heads, size_t head_dim, size_t tk,
                                 size_t cap, float scale, int scale_q, llmtie_decode_scratch* scratch, float* out,
                                 size_t out_len, int8_t* twin, size_t twin_rows, size_t twin_k, size_t row);

/* flash_attn_f16 (device.rs:5754) off the tiled cache. */
int llmtie_flash_attn_t16(void* stream, const float* q, size_t q_len, const uint16_t* cache, size_t cache_len,
                          float* out, size_t out_len, size_t tq, size_t past, size_t heads, size_t kv_heads,
                          size_t head_dim, size_t cap, float scale, int causal);

/* --------------------------------------------------------- KV producers */

/* Gpu::rope / rope_scaled (device.rs:5410, :5430; kernel kernels.rs:4915): in place over x[off ..] of
 * [t, heads*head_dim]; freq_div (head_dim/2 floats, device) may be NULL. */
int llmtie_rope(void* stream, float* x, size_t x_len, size_t off, const float* freq_div, size_t t, size_t heads,
                size_t head_dim, float theta, size_t first);

/* Gpu::cache_append / cache_append_f16 (device.rs:3013 / :2849): n rows of
 * src[src_off ..] ([n, kv_heads*head_dim]) into positions past.. of a cache;
 * transposed selects the V layout. */
int llmtie_cache_append(void* stream, const float* src, size_t src_len, size_t src_off, float* dst, size_t dst_len,
                        size_t n, size_t kv_heads, size_t head_dim, size_t cap, size_t past, int transposed);
int llmtie_cache_append_f16(void* stream, const float* src, size_t src_len, size_t src_off, uint16_t* dst,
                            size_t dst_len, size_t n, size_t kv_heads, size_t head_dim, size_t cap, size_t past,
                            int transposed);

/* Gpu::rope_cache_f16 (device.rs:2915): q rotated in place, k rotated and v
 * stored into the f16 caches at `pos`. */
int llmtie_rope_cache_f16(void* stream, float* q, size_t q_len, size_t q_off, const float* k, size_t k_len,
                          size_t k_off, const float* v, size_t v_len, size_t v_off, const float* freq_div,
                          size_t heads, size_t kv_heads, size_t head_dim, float theta, size_t pos, uint16_t* kc,
                          uint16_t* vc, size_t cache_len, size_t cap);

/* Gpu::cache_grow / cache_grow_f16 (device.rs:3086, :3152): re-stride the first
 * `live` positions of every head from capacity cap to new_cap. */
int llmtie_cache_grow(void* stream, const float* src, size_t src_len, float* dst, size_t dst_len, size_t kv_heads,
                      size_t head_dim, size_t cap, size_t new_cap, size_t live, int transposed);
int llmtie_cache_grow_f16(void* stream, const uint16_t* src, size_t src_len, uint16_t* dst, size_t dst_len,
                          size_t kv_heads, size_t head_dim, size_t cap, size_t new_cap, size_t live,
                          int transposed);

/* Bytes a tiled Q8_0 cache of this shape holds (layout at the top). */
size_t llmtie_q8_cache_bytes(size_t slots, size_t kv_heads, size_t head_dim, size_t cap);

/* Q8_0 cache append (new): n rows of k[k_off..] and v[v_off..] ([n,
 * kv_heads*head_dim], k already rotated) quantized into slot `slot` at
 * positions past.. . Quantization is ggml's quantize_row_q8_0_ref. */
int llmtie_kv_q8_append(void* stream, const float* k, size_t k_len, size_t k_off, const float* v, size_t v_len,
                        size_t v_off, int8_t* cache, size_t cache_len, size_t slots, size_t slot, size_t n,
                        size_t kv_heads, size_t head_dim, size_t cap, size_t past);

/* The Q8_0 twin of llmtie_rope_cache_f16 (new): q rotated in place, k rotated
 * and quantized, v quantized, into slot `slot` at `pos`. */
int llmtie_rope_cache_q8(void* stream, float* q, size_t q_len, size_t q_off, const float* k, size_t k_len,
                         size_t k_off, const float* v, size_t v_len, size_t v_off, const float* freq_div,
                         size_t heads, size_t kv_heads, size_t head_dim, float theta, size_t pos, int8_t* cache,
                         size_t cache_len, size_t slots, size_t slot, size_t cap);

#ifdef __cplusplus
}
#endif

#endif /* LLMTIE_HIP_H */
