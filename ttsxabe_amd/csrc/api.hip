// The C ABI (include/llmtie_hip.h): argument checks in the reference's order
// and with its error variants, then one launch. Mirrors the `impl Gpu`
// attention methods of crates/llmtie-cuda/src/device.rs:5697-6410 and the
// cache producers at :2849-3190, :5410-5470.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <mutex>
#include <vector>

#include "../../include/llmtie_hip.h"
#include "decode.h"
#include "kvlayout.h"
#include "kvcache.h"
#include "prefill.h"

using namespace llmtie;

namespace {

thread_local llmtie_error g_err = {0, {0, 0, 0, 0}, {0}};
// llmtie_debug_fake_xcc: the test hook for the XCD-local check.
std::atomic<bool> g_fake_xcc{false};

int fail(int status, size_t f0, size_t f1, size_t f2, size_t f3, const char* fmt, ...) {
    g_err.status = status;
    g_err.field[0] = f0;
    g_err.field[1] = f1;
    g_err.field[2] = f2;
    g_err.field[3] = f3;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err.message, sizeof g_err.message, fmt, ap);
    va_end(ap);
    return status;
}

int ok() {
    g_err.status = LLMTIE_OK;
    g_err.message[0] = 0;
    return LLMTIE_OK;
}

int unsupported(size_t hd, size_t heads, size_t kv) {
    return fail(LLMTIE_UNSUPPORTED_ATTENTION, hd, heads, kv, 0,
                "fused attention wants head_dim 64 or 128 and heads a multiple of kv_heads, got head_dim %zu, "
                "%zu heads over %zu",
                hd, heads, kv);
}
int overrun_slice(size_t at, size_t len) {
    return fail(LLMTIE_SLICE_OVERRUN, at, len, 0, 0, "reading to %zu in a buffer of %zu", at, len);
}
int overrun_cache(size_t at, size_t cap) {
    return fail(LLMTIE_CACHE_OVERRUN, at, cap, 0, 0, "appending at %zu to a cache with room for %zu", at, cap);
}
int odd_cap(size_t cap) {
    return fail(LLMTIE_ODD_CACHE_CAPACITY, cap, 0, 0, 0, "an f16 cache with an odd capacity of %zu", cap);
}
int invalid(const char* what) { return fail(LLMTIE_INVALID_ARGUMENT, 0, 0, 0, 0, "%s is null", what); }
int driver(const char* what, hipError_t e) {
    if (e == hipErrorNoDevice || e == hipErrorInsufficientDriver)
        return fail(LLMTIE_NO_DEVICE, 0, 0, 0, 0, "no usable HIP device: %s", hipGetErrorString(e));
    return fail(LLMTIE_DRIVER, (size_t)e, 0, 0, 0, "%s: %s", what, hipGetErrorString(e));
}
int launched(const char* what, hipError_t e) { return e == hipSuccess ? ok() : driver(what, e); }

hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Every kernel takes int extents; anything that does not fit is refused as
// an overrun of the int range rather than silently wrapped.
constexpr size_t IMAX = 0x7fffffff;

// Sizes computed from caller arguments saturate at SIZE_MAX instead of
// wrapping, so a length check on a sum or product never passes on overflow.
size_t smul(size_t a, size_t b) {
    size_t r;
    return __builtin_mul_overflow(a, b, &r) ? SIZE_MAX : r;
}
size_t smul(size_t a, size_t b, size_t c) { return smul(smul(a, b), c); }
size_t sadd(size_t a, size_t b) {
    size_t r;
    return __builtin_add_overflow(a, b, &r) ? SIZE_MAX : r;
}
// The first of up to four counts that does not fit an int, refused as an
// overrun of the int range (0 when all fit).
int over_int(size_t a, size_t b = 0, size_t c = 0, size_t d = 0) {
    const size_t m = std::max(std::max(a, b), std::max(c, d));
    return m > IMAX ? overrun_slice(m, IMAX) : 0;
}

}  // namespace

struct llmtie_decode_scratch {
    float* part = nullptr;
    size_t part_cap = 0;  // floats
    unsigned* ctr = nullptr;
    size_t ctr_cap = 0;   // counters
    int device = -1;
    // Buffers replaced by growth. A HIP graph captured with the scratch keeps
    // their addresses, so they stay allocated until the scratch is freed.
    std::vector<void*> retired;
    // Host-visible word (pinned host memory) the decode kernel sets when an
    // XCD-local head's split workgroups turn out not to share an XCD.
    unsigned* lost = nullptr;
};

extern "C" {

int llmtie_last_error(llmtie_error* out) {
    if (out) *out = g_err;
    return g_err.status;
}

const char* llmtie_version(void) { return "0.1.0"; }

llmtie_decode_scratch* llmtie_decode_scratch_new(void) { return new llmtie_decode_scratch(); }

void llmtie_decode_scratch_free(llmtie_decode_scratch* s) {
    if (!s) return;
    if (s->part) (void)hipFree(s->part);
    if (s->ctr) (void)hipFree(s->ctr);
    for (void* p : s->retired) (void)hipFree(p);
    if (s->lost) (void)hipHostFree(s->lost);
    delete s;
}

int llmtie_decode_scratch_status(llmtie_decode_scratch* s) {
    if (!s || !s->lost || !__atomic_load_n(s->lost, __ATOMIC_ACQUIRE)) return LLMTIE_OK;
    __atomic_store_n(s->lost, 0u, __ATOMIC_RELEASE);
    return fail(LLMTIE_SPLIT_HEAD_LOST, 0, 0, 0, 0,
                "an earlier decode through this scratch wrote NaN for a head whose split workgroups did not "
                "share an XCD; LLMTIE_DECODE_XCD=0 selects the coherent hand-off");
}

void llmtie_debug_fake_xcc(int on) { g_fake_xcc.store(on != 0); }

int llmtie_supports_flash(size_t head_dim, size_t heads, size_t kv_heads) {
    return (head_dim == 64 || head_dim == 128) && kv_heads > 0 && heads % kv_heads == 0 && heads > 0;
}

}  // extern "C"

namespace {

int compute_units();

// 16-query tiles per wave: the most that still leaves about two workgroups
// per CU (256 CUs), so short prefills spread over the whole chip.
int pick_nqt(size_t tq, size_t heads, int gb, bool staged = false) {
    if (const char* e = getenv("LLMTIE_PREFILL_NQT")) {
        const int v = atoi(e);
        if (v == 1 || v == 2 || v == 4) return v;
    }
    // Measured on MI355X (C3 shapes, 512 to 8192 rows): two 16-row query
    // tiles per wave (each K/V fragment read from LDS feeds two MFMAs) win
    // once the launch still has >= 512 workgroups; below that, one tile per
    // wave, for the parallelism.
    const size_t pb2 = 32 * (4 / gb);
    const size_t wg2 = ((tq + pb2 - 1) / pb2) * (heads / gb);
    if (wg2 >= 512) return 2;
    // f32 sources staged through registers: two tiles per wave halve the
    // staging per query row, which wins down to about one workgroup per CU
    // (the encoder rows at 240 workgroups: 38.7 vs 40.1 us, before their
    // eight-wave kernel).
    if (staged && wg2 >= 192) return 2;
    return 1;
}

int prefill_common(void* stream, int kind, const float* q, size_t q_len, const void* k, size_t k_len, const void* v,
                   size_t v_len, float* out, size_t out_len, size_t tq, size_t past, size_t heads, size_t kv_heads,
                   size_t hd, size_t cap, float scale, int causal) {
    if (!(hd == 64 || hd == 128) || kv_heads == 0 || heads % kv_heads != 0) return unsupported(hd, heads, kv_heads);
    if (sadd(past, tq) > cap) return overrun_cache(sadd(past, tq), cap);
    if (int r = over_int(smul(heads, hd), cap)) return r;
    const size_t nq = smul(tq, heads, hd);
    if (nq > (size_t)1 << 40) return overrun_slice(nq, (size_t)1 << 40);
    if (q_len < nq) return overrun_slice(nq, q_len);
    const size_t need = smul(kv_heads, cap, hd);
    if (k_len < need || v_len < need) return overrun_slice(need, std::min(k_len, v_len));
    if (out_len < nq) return overrun_slice(nq, out_len);
    if (tq == 0) return ok();
    if (!q || !k || !v || !out) return invalid("a buffer");
    const size_t group = heads / kv_heads;
    const int gb = group % 4 == 0 ? 4 : (group % 2 == 0 ? 2 : 1);
    PrefillArgs a{};
    a.cus = compute_units();
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.tq = (int)tq;
    a.past = (int)past;
    a.heads = (int)heads;
    a.kv_heads = (int)kv_heads;
    a.cap = (int)cap;
    a.scale = scale;
    a.causal = causal ? 1 : 0;
    a.gb = gb;
    a.qs = (int)(heads * hd);
    a.kvs = 0;
    a.os = (int)(heads * hd);
    a.scale_q = 0;
    a.v_bytes = v_len * (kind == PF_F32 ? 4 : 2);
    const int nqt = pick_nqt(tq, heads, gb, kind == PF_F32);
    return launched("flash_attn", launch_prefill((int)hd, kind, nqt, a, S(stream)));
}

// Compute units of the current device (cached per device).
int compute_units() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// Splits of one head: about `target` workgroups over the whole launch, each
// wave taking whole 32-key blocks, and never more than the merge can hold.
void plan_decode(size_t tk_max, size_t units, size_t group, int& nit, int& splits) {
    const size_t max_splits = std::min<size_t>(DECODE_MAX_SPLITS, DECODE_MAX_SPLIT_ROWS / std::max<size_t>(1, group));
    // Measured on MI355X: a lone sequence decodes fastest over ~256
    // workgroups (C2: 10.99 us at 128, 10.69 at 256, flat beyond; with the
    // arrival counters on separate lines the in-launch merge no longer grows
    // costlier with the split count); a batch wants about three splits per
    // (sequence, kv head) at its longest context so the long sequences do not
    // set the time alone.
    size_t target = std::max<size_t>(256, 3 * units);
    if (const char* e = getenv("LLMTIE_DECODE_WGS")) target = std::max(1, atoi(e));
    const size_t blocks = (tk_max + 31) / 32;
    size_t want = std::max<size_t>(1, target / std::max<size_t>(1, units));
    size_t per_wg = (blocks + want - 1) / want;           // 32-key blocks per workgroup
    size_t n = std::max<size_t>(1, (per_wg + 3) / 4);     // per wave
    if (const char* e = getenv("LLMTIE_DECODE_NIT")) n = std::max(1, atoi(e));
    // A short context is one split: the cross-workgroup merge (three memory
    // round trips, ~3 us) costs more than the extra parallelism saves below
    // ~12 blocks per head (measured: 224 keys 9.2 us unsplit vs 12.4 us in
    // two splits; 512 keys 10.7 us unsplit vs 10.0 us in two).
    if (blocks <= 12 && !getenv("LLMTIE_DECODE_WGS") && !getenv("LLMTIE_DECODE_NIT")) n = (blocks + 3) / 4;
    size_t span = 4 * n * 32;
    while ((tk_max + span - 1) / span > max_splits) {
        ++n;
        span = 4 * n * 32;
    }
    nit = (int)n;
    splits = (int)((tk_max + span - 1) / span);
}

// Whether the split partials are merged by a second launch rather than by
// the last-arriving workgroup of each head.
int two_phase_merge(int splits, size_t units) {
    if (const char* e = getenv("LLMTIE_DECODE_TWO_PHASE")) return atoi(e) ? 1 : 0;
    // The in-launch hand-off (coherent stores, a wait, an atomic per
    // workgroup, each counter on its own line) measured faster than a second
    // launch up to 512 workgroups (C2 at 256: 10.69 vs 12.12 us); a second
    // launch merges beyond 1024.
    return (size_t)splits * units > 1024 ? 1 : 0;
}

// Floats of the (m, l) area per (sequence, kv head): whole 256-byte lines,
// so no line is shared by two heads' partials.
size_t ml_stride(int splits, size_t group) { return ((size_t)splits * group * 2 + 63) / 64 * 64; }

// Whether a host-planned in-launch merge keeps every head on one XCD: the
// dispatcher deals a launch's workgroups to the eight XCDs of gfx950 in
// turn, so workgroups L and L + 8k share an XCD (which XCD a launch starts on
// varies with what ran before; a partitioned device with fewer XCDs still
// groups them). The plan runs workgroup L on item (L % 8) * (launch / 8) +
// L / 8, so each XCD's run of items must hold whole heads. The kernel checks
// the grouping itself (the arrival counter sums the XCC ids).
int xcd_local(int splits, size_t units, int two_phase) {
    if (const char* e = getenv("LLMTIE_DECODE_XCD")) {
        if (!atoi(e)) return 0;
    }
    const size_t total = (size_t)splits * units;
    if (two_phase || splits <= 1 || total % 8 != 0) return 0;
    return (total / 8) % (size_t)splits == 0 ? 1 : 0;
}

// A buffer the scratch no longer uses. It is kept allocated until the
// scratch is freed: a graph captured earlier may still read it. (Growth is by
// powers of two, so a scratch retires a few dozen buffers at most.)
int retire(llmtie_decode_scratch* s, void* p) {
    if (p) s->retired.push_back(p);
    return LLMTIE_OK;
}

int ensure_scratch(llmtie_decode_scratch* s, size_t part_floats, size_t ctrs, hipStream_t st) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return driver("hipGetDevice", e);
    const bool swap = s->device != dev;
    const bool grow = swap || s->part_cap < part_floats || s->ctr_cap < ctrs;
    if (!grow) return LLMTIE_OK;
    // Allocating inside a stream capture would put the allocation into the
    // graph (or fail); the caller makes one eager call first instead.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(st, &cs);
    if (e != hipSuccess) return driver("hipStreamIsCapturing", e);
    if (cs != hipStreamCaptureStatusNone)
        return fail(LLMTIE_SCRATCH_GROWTH_IN_CAPTURE, part_floats, s->part_cap, ctrs, s->ctr_cap,
                    "the decode scratch must grow to %zu partial floats and %zu counters while the stream is "
                    "capturing a graph; make one call of this shape before capturing",
                    part_floats, ctrs);
    int r;
    if (swap) {
        // A scratch follows the device it is used on; switching starts over.
        if ((r = retire(s, s->part)) != LLMTIE_OK || (r = retire(s, s->ctr)) != LLMTIE_OK) return r;
        s->part = nullptr;
        s->ctr = nullptr;
        s->part_cap = s->ctr_cap = 0;
        s->device = dev;
    }
    if (!s->lost) {
        void* w = nullptr;
        e = hipHostMalloc(&w, sizeof(unsigned), hipHostMallocMapped | hipHostMallocCoherent);
        if (e != hipSuccess) return driver("allocating the scratch's status word", e);
        s->lost = static_cast<unsigned*>(w);
        *s->lost = 0;
    }
    if (s->part_cap < part_floats) {
        size_t want = 1024;
        while (want < part_floats) want <<= 1;
        float* p = nullptr;
        e = hipMalloc(&p, want * sizeof(float));
        if (e != hipSuccess) return driver("allocating", e);
        if ((r = retire(s, s->part)) != LLMTIE_OK) {
            (void)hipFree(p);
            return r;
        }
        s->part = p;
        s->part_cap = want;
    }
    if (s->ctr_cap < ctrs) {
        size_t want = 64;
        while (want < ctrs) want <<= 1;
        unsigned* c = nullptr;
        e = hipMalloc(&c, want * sizeof(unsigned));
        if (e != hipSuccess) return driver("allocating", e);
        // Zeroed by a kernel on the caller's stream (a memset node inside a
        // captured graph is not to be relied on).
        e = launch_fill_u32(c, want, 0u, st);
        if (e != hipSuccess) {
            (void)hipFree(c);
            return driver("zeroing", e);
        }
        if ((r = retire(s, s->ctr)) != LLMTIE_OK) return r;
        s->ctr = c;
        s->ctr_cap = want;
    }
    return LLMTIE_OK;
}

// Partials and counters of the no-allocation decode (device addresses).
struct FixedScratch {
    float* part;
    size_t part_cap;  // floats
    unsigned* ctr;
    size_t ctr_cap;   // words
};

// Sizes of the no-allocation decode's fixed scratch: split partials, then
// arrival counters (CTR_STRIDE words per kv head).
constexpr size_t NOALLOC_PART_FLOATS = (size_t)1 << 20;
constexpr size_t NOALLOC_CTR_WORDS = (size_t)256 * CTR_STRIDE;
int noalloc_scratch(hipStream_t st, FixedScratch& f);

// The checks and the launch behind every single-sequence decode
// (device.rs:6224-6410).
int decode_common(void* stream, int kind, const float* q, size_t q_len, size_t q_off, const void* k, size_t k_len,
                  const void* v, size_t v_len, size_t heads, size_t kv_heads, size_t hd, size_t tk, size_t cap,
                  float scale, int scale_q, llmtie_decode_scratch* scratch, float* out, size_t out_len,
                  size_t out_off, int8_t* twin, size_t twin_rows, size_t twin_k, bool has_twin,
                  bool noalloc = false) {
    const bool tiled = kind == KV_T16;
    if (!(hd == 64 || hd == 128)) return unsupported(hd, heads, kv_heads);
    if (kv_heads == 0 || heads % kv_heads != 0 || heads / kv_heads > 16) return unsupported(hd, heads, kv_heads);
    if (tk == 0 || tk > cap) return overrun_cache(tk, cap);
    const size_t esz = kind == KV_F32 ? 4 : 2;
    if (!tiled && (cap * esz) % 8 != 0) return odd_cap(cap);
    if (int r = over_int(cap, heads)) return r;
    if (smul(kv_heads, cap, hd) > ((size_t)1 << 40)) return overrun_slice(smul(kv_heads, cap, hd), (size_t)1 << 40);
    if (tiled) {
        const size_t need = kv_heads * (size_t)tiled_nblk((int)cap) * 64 * hd;
        if (k_len < need) return overrun_slice(need, k_len);
        v = k;
    } else {
        const size_t need = kv_heads * cap * hd;
        if (k_len < need || v_len < need) return overrun_slice(need, std::min(k_len, v_len));
    }
    const size_t n = heads * hd;
    if (q_len < sadd(q_off, n)) return overrun_slice(sadd(q_off, n), q_len);
    if (out_len < sadd(out_off, n)) return overrun_slice(sadd(out_off, n), out_len);
    if (out_off % 32 != 0) return fail(LLMTIE_RAGGED_BLOCK, out_off, 32, 0, 0, "a row of %zu in blocks of 32", out_off);
    if (has_twin) {
        // The scales follow the codes at twin + twin_rows * twin_k.
        if (int r = over_int(twin_rows)) return r;
        if (twin_k != n || smul(twin_rows, twin_k) < out_off + n)
            return fail(LLMTIE_MISMATCHED_Q8, twin_rows, twin_k, out_off / n + 1, n,
                        "an int8 twin of %zu rows by %zu where %zu by %zu is needed", twin_rows, twin_k,
                        out_off / n + 1, n);
        if (!twin) return invalid("twin");
    }
    if (!q || !k || !v || !out) return invalid("a buffer");
    if (!scratch && !noalloc) return invalid("scratch");
    // A head lost by an earlier call through this scratch (see
    // llmtie_decode_scratch_status) is reported before anything is launched.
    if (!noalloc) {
        if (int r = llmtie_decode_scratch_status(scratch)) return r;
    }
    const size_t group = heads / kv_heads;
    int nit, splits;
    plan_decode(tk, kv_heads, group, nit, splits);
    const size_t mls = ml_stride(splits, group);
    const size_t part = kv_heads * ((size_t)splits * group * hd + mls);
    const long ml_off = (long)(kv_heads * (size_t)splits * group * hd);
    float* part_p;
    unsigned* ctr_p;
    if (noalloc) {
        // Refused before the device is touched.
        if (part > NOALLOC_PART_FLOATS || kv_heads * CTR_STRIDE > NOALLOC_CTR_WORDS)
            return fail(LLMTIE_SCRATCH_LIMIT, part, NOALLOC_PART_FLOATS, kv_heads * CTR_STRIDE, NOALLOC_CTR_WORDS,
                        "the call needs %zu partial floats and %zu counter words; the fixed scratch holds %zu and "
                        "%zu",
                        part, kv_heads * CTR_STRIDE, NOALLOC_PART_FLOATS, NOALLOC_CTR_WORDS);
        FixedScratch f;
        int r = noalloc_scratch(S(stream), f);
        if (r != LLMTIE_OK) return r;
        part_p = f.part;
        ctr_p = f.ctr;
    } else {
        int r = ensure_scratch(scratch, part, kv_heads * CTR_STRIDE, S(stream));
        if (r != LLMTIE_OK) return r;
        part_p = scratch->part;
        ctr_p = scratch->ctr;
    }
    DecodeArgs a;
    memset(&a, 0, sizeof a);
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    if (has_twin) {
        a.twin_codes = twin;
        a.twin_scales = reinterpret_cast<float*>(twin + twin_rows * twin_k);
    }
    a.part = part_p;
    a.ml_off = ml_off;
    a.ctr = ctr_p;
    a.q_off = (long)q_off;
    a.out_off = (long)out_off;
    a.tk = (int)tk;
    a.cap = (int)cap;
    a.kv_heads = (int)kv_heads;
    a.group = (int)group;
    a.score_l2 = (scale_q ? 1.0f : scale) * 1.4426950408889634f;
    a.qscale = scale_q ? scale : 1.0f;
    a.nit = nit;
    a.splits = splits;
    a.ml_stride = (long)mls;
    a.two_phase = two_phase_merge(splits, kv_heads);
    // The no-allocation path has no status word to report a lost head to,
    // so it always hands partials over coherently.
    a.xcd = noalloc ? 0 : xcd_local(splits, kv_heads, a.two_phase);
    a.xcd_fake = g_fake_xcc.load() ? 1 : 0;
    a.lost = noalloc ? nullptr : scratch->lost;
    return launched("attn_decode", launch_decode((int)hd, kind, a, (int)kv_heads, 1, S(stream)));
}

}  // namespace

extern "C" {

int llmtie_flash_attn(void* stream, const float* q, size_t q_len, const float* k, size_t k_len, const float* v,
                      size_t v_len, float* out, size_t out_len, size_t tq, size_t past, size_t heads,
                      size_t kv_heads, size_t head_dim, size_t cap, float scale, int causal) {
    return prefill_common(stream, PF_F32, q, q_len, k, k_len, v, v_len, out, out_len, tq, past, heads, kv_heads,
                          head_dim, cap, scale, causal);
}

int llmtie_flash_attn_f16(void* stream, const float* q, size_t q_len, const uint16_t* k, size_t k_len,
                          const uint16_t* v, size_t v_len, float* out, size_t out_len, size_t tq, size_t past,
                          size_t heads, size_t kv_heads, size_t head_dim, size_t cap, float scale, int causal) {
    if (!(head_dim == 64 || head_dim == 128)) return unsupported(head_dim, heads, kv_heads);
    if (cap % 2 != 0) return odd_cap(cap);
    return prefill_common(stream, PF_F16, q, q_len, k, k_len, v, v_len, out, out_len, tq, past, heads, kv_heads,
                          head_dim, cap, scale, causal);
}

int llmtie_flash_attn_rows(void* stream, const float* qkv, size_t qkv_len, uint16_t* out, size_t out_len, size_t t,
                           size_t heads, size_t head_dim, float scale) {
    if (head_dim != 64 || heads == 0) return unsupported(head_dim, heads, heads);
    if (int r = over_int(smul(heads, head_dim, 3), t)) return r;
    const size_t d = heads * head_dim;
    if (qkv_len < smul(t, 3 * d)) return overrun_slice(smul(t, 3 * d), qkv_len);
    if (out_len < smul(t, d)) return overrun_slice(smul(t, d), out_len);
    if (t == 0) return ok();
    if (!qkv || !out) return invalid("a buffer");
    PrefillArgs a{};
    a.cus = compute_units();
    a.q = qkv;
    a.k = qkv + d;
    a.v = qkv + 2 * d;
    a.out = out;
    a.tq = (int)t;
    a.past = 0;
    a.heads = (int)heads;
    a.kv_heads = (int)heads;
    a.cap = (int)t;
    a.scale = scale;
    a.causal = 0;
    a.gb = 1;
    a.qs = (int)(3 * d);
    a.kvs = (int)(3 * d);
    a.os = (int)d;
    a.scale_q = 1;
    a.out_f16 = 1;
    // The stacked f32 rows are read in place: the attention kernel stages
    // them through registers into its f16 LDS tiles (no copy, no workspace).
    // Eight-wave workgroups of one query tile per wave: the staging per row
    // of two tiles per wave, at two waves per SIMD (C4 encoder 38.2 -> 35.8
    // us). LLMTIE_ROWS_W8=0 selects the four-wave kernel.
    const char* w8 = getenv("LLMTIE_ROWS_W8");
    if (!(w8 && !atoi(w8))) return launched("flash_attn_rows", launch_prefill(64, PF_ROWS, 1, a, S(stream), 8));
    return launched("flash_attn_rows", launch_prefill(64, PF_ROWS, pick_nqt(t, heads, 1, true), a, S(stream)));
}

int llmtie_attn_decode_f16(void* stream, const float* q, size_t q_len, const uint16_t* k, size_t k_len,
                           const uint16_t* v, size_t v_len, size_t heads, size_t kv_heads, size_t head_dim,
                           size_t tk, size_t cap, float scale, int scale_q, llmtie_decode_scratch* scratch,
                           float* out, size_t out_len) {
    return decode_common(stream, KV_F16, q, q_len, 0, k, k_len, v, v_len, heads, kv_heads, head_dim, tk, cap, scale,
                         scale_q, scratch, out, out_len, 0, nullptr, 0, 0, false);
}

}  // extern "C"

// ------------------------------------------------ decode without allocation
//
// `scratch`: the split partials (NOALLOC_PART_FLOATS floats) then the arrival
// counters (NOALLOC_CTR_WORDS words, CTR_STRIDE per kv head) of
// llmtie_attn_decode_f16_noalloc, 4.25 MiB held on every device the library
// runs on until the process ends. Host code never passes the array's name
// (a host-side stand-in, not a device address) to the device: it uses the
// address hipGetSymbolAddress gives for the current device, obtained once per
// device.
static __device__ __align__(256) float scratch[NOALLOC_PART_FLOATS + NOALLOC_CTR_WORDS];

namespace {

std::mutex noalloc_mu;
float* noalloc_ptr[64];

// This device's copy of `scratch` (zero at load; every call leaves its
// counters at zero).
int noalloc_scratch(hipStream_t st, FixedScratch& f) {
    (void)st;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return driver("hipGetDevice", e);
    if (dev < 0 || dev >= 64) return driver("device index", hipErrorInvalidDevice);
    std::lock_guard<std::mutex> lock(noalloc_mu);
    if (!noalloc_ptr[dev]) {
        float* p = nullptr;
        e = hipGetSymbolAddress(reinterpret_cast<void**>(&p), HIP_SYMBOL(scratch));
        if (e != hipSuccess) return driver("hipGetSymbolAddress(scratch)", e);
        // No clearing launch: the array has no initialiser, so it is zero
        // when the code object is loaded (a zero-filled segment), and every
        // call leaves its counters at zero. A fill here would be recorded
        // into a graph if this first call were made under stream capture.
        noalloc_ptr[dev] = p;
    }
    f.part = noalloc_ptr[dev];
    f.part_cap = NOALLOC_PART_FLOATS;
    f.ctr = reinterpret_cast<unsigned*>(noalloc_ptr[dev] + NOALLOC_PART_FLOATS);
    f.ctr_cap = NOALLOC_CTR_WORDS;
    return LLMTIE_OK;
}

}  // namespace

extern "C" {

int llmtie_attn_decode_f16_noalloc(void* stream, const float* q, size_t q_len, const uint16_t* k, size_t k_len,
                                   const uint16_t* v, size_t v_len, size_t heads, size_t kv_heads, size_t head_dim,
                                   size_t tk, size_t cap, float scale, int scale_q, float* out, size_t out_len) {
    return decode_common(stream, KV_F16, q, q_len, 0, k, k_len, v, v_len, heads, kv_heads, head_dim, tk, cap, scale,
                         scale_q, nullptr, out, out_len, 0, nullptr, 0, 0, false, true);
}

int llmtie_attn_decode_f16_q(void* stream, const float* q, size_t q_len, const uint16_t* k, size_t k_len,
                             const uint16_t* v, size_t v_len, size_t heads, size_t kv_heads, size_t head_dim,
                             size_t tk, size_t cap, float scale, int scale_q, llmtie_decode_scratch* scratch,
                             float* out, size_t out_len, int8_t* twin, size_t twin_len) {
    const size_t n = smul(heads, head_dim);
    if (twin_len < sadd(n, (n / 32) * 4)) return overrun_slice(sadd(n, (n / 32) * 4), twin_len);
    if (n % 32 != 0) return fail(LLMTIE_RAGGED_BLOCK, n, 32, 0, 0, "a row of %zu in blocks of 32", n);
    return decode_common(stream, KV_F16, q, q_len, 0, k, k_len, v, v_len, heads, kv_heads, head_dim, tk, cap, scale,
                         scale_q, scratch, out, out_len, 0, twin, 1, n, true);
}

int llmtie_attn_decode_f16_q_row(void* stream, const float* q, size_t q_len, size_t q_off, const uint16_t* k,
                                 size_t k_len, const uint16_t* v, size_t v_len, size_t heads, size_t kv_heads,
                                 size_t head_dim, size_t tk, size_t cap, float scale, int scale_q,
                                 llmtie_decode_scratch* scratch, float* out, size_t out_len, int8_t* twin,
                                 size_t twin_rows, size_t twin_k, size_t row) {
    return decode_common(stream, KV_F16, q, q_len, q_off, k, k_len, v, v_len, heads, kv_heads, head_dim, tk, cap,
                         scale, scale_q, scratch, out, out_len, smul(row, heads, head_dim), twin, twin_rows, twin_k,
                         true);
}

int llmtie_attn_decode(void* stream, const float* q, size_t q_len, const float* k, size_t k_len, const float* v,
                       size_t v_len, size_t heads, size_t kv_heads, size_t head_dim, size_t tk, size_t cap,
                       float scale, int scale_q, llmtie_decode_scratch* scratch, float* out, size_t out_len) {
    return decode_common(stream, KV_F32, q, q_len, 0, k, k_len, v, v_len, heads, kv_heads, head_dim, tk, cap, scale,
                         scale_q, scratch, out, out_len, 0, nullptr, 0, 0, false);
}

int llmtie_attn_decode_q8_batch(void* stream, const float* q, size_t q_len, const int8_t* cache, size_t cache_len,
                                size_t slots, const int32_t* tk_dev, const int32_t* slot_dev, size_t nseq,
                                size_t max_tk, size_t heads, size_t kv_heads, size_t head_dim, size_t cap,
                                float scale, int scale_q, llmtie_decode_scratch* scratch, float* out,
                                size_t out_len) {
    if (!(head_dim == 64 || head_dim == 128)) return unsupported(head_dim, heads, kv_heads);
    // Groups are bounded by the stream-K kernel's LDS (sk_group_max: 16 at
    // head_dim 64 and 128).
    if (kv_heads == 0 || heads % kv_heads != 0 || heads / kv_heads > (size_t)sk_group_max((int)head_dim))
        return unsupported(head_dim, heads, kv_heads);
    if (max_tk == 0 || max_tk > cap) return overrun_cache(max_tk, cap);
    if (nseq > 65535) return overrun_slice(nseq, 65535);
    // The stream-K kernel addresses one (slot, kv head)'s blocks through a
    // 32-bit buffer range.
    if (smul((cap + 31) / 32, sk_block_bytes((int)head_dim)) > 0x7fffffffu) return overrun_cache(cap, 0x7fffffffu / sk_block_bytes((int)head_dim) * 32);
    if (int r = over_int(cap, slots, heads)) return r;
    const size_t need = llmtie_q8_cache_bytes(slots, kv_heads, head_dim, cap);
    if (cache_len < need) return overrun_slice(need, cache_len);
    const size_t n = heads * head_dim;
    if (q_len < nseq * n) return overrun_slice(nseq * n, q_len);
    if (out_len < nseq * n) return overrun_slice(nseq * n, out_len);
    if (nseq == 0) return ok();
    if (!q || !cache || !tk_dev || !slot_dev || !out) return invalid("a buffer");
    if (!scratch) return invalid("scratch");
    if (int r = llmtie_decode_scratch_status(scratch)) return r;
    const size_t group = heads / kv_heads;
    int nit, splits;
    plan_decode(max_tk, kv_heads * nseq, group, nit, splits);
    // Up to 64 sequences go through the stream-K kernel, one workgroup per
    // compute unit, each wave an equal share of the batch's blocks; a larger
    // batch through the host-planned grid (splits of the longest sequence).
    const bool sk = nseq <= 64 && !getenv("LLMTIE_DECODE_STATIC");
    const int items = sk ? compute_units() : 0;
    const size_t mls = ml_stride(splits, group);
    size_t part = nseq * kv_heads * ((size_t)splits * group * head_dim + mls);
    long ml_off = (long)(nseq * kv_heads * (size_t)splits * group * head_dim);
    if (sk) {
        const size_t slots2 = (size_t)items * SK_WAVES * 2;
        ml_off = (long)(slots2 * 16 * head_dim);
        part = slots2 * (16 * head_dim + 32);
    }
    int r = ensure_scratch(scratch, part, nseq * kv_heads * CTR_STRIDE, S(stream));
    if (r != LLMTIE_OK) return r;
    DecodeArgs a;
    memset(&a, 0, sizeof a);
    a.q = q;
    a.k = cache;
    a.out = out;
    a.part = scratch->part;
    a.ml_off = ml_off;
    a.ctr = scratch->ctr;
    a.tk_arr = tk_dev;
    a.slot_arr = slot_dev;
    a.q_stride = (long)n;
    a.out_stride = (long)n;
    a.tk = (int)max_tk;
    a.slots = (int)slots;
    a.cap = (int)cap;
    a.kv_heads = (int)kv_heads;
    a.group = (int)group;
    a.score_l2 = (scale_q ? 1.0f : scale) * 1.4426950408889634f;
    a.qscale = scale_q ? scale : 1.0f;
    a.nit = nit;
    a.splits = splits;
    a.ml_stride = (long)mls;
    a.two_phase = sk ? 0 : two_phase_merge(splits, kv_heads * nseq);
    a.xcd = sk ? 0 : xcd_local(splits, kv_heads * nseq, a.two_phase);
    a.xcd_fake = g_fake_xcc.load() ? 1 : 0;
    a.lost = scratch->lost;
    a.sk = sk ? 1 : 0;
    a.nseq = (int)nseq;
    a.items = items;
    return launched("attn_decode_q8_batch", launch_decode((int)head_dim, KV_TQ8, a, (int)kv_heads, (int)nseq, S(stream)));
}

int llmtie_rope(void* stream, float* x, size_t x_len, size_t off, const float* freq_div, size_t t, size_t heads,
                size_t head_dim, float theta, size_t first) {
    if (int r = over_int(t, heads, head_dim, first)) return r;
    const size_t nx = smul(t, heads, head_dim);
    if (sadd(off, nx) > x_len) return overrun_slice(sadd(off, nx), x_len);
    if (head_dim % 2 != 0) return fail(LLMTIE_ODD_HEAD_DIM, head_dim, 0, 0, 0, "a rotary head of odd width %zu", head_dim);
    if (nx == 0) return ok();
    if (!x) return invalid("x");
    return launched("rope", launch_rope(x, (long)off, freq_div, (int)t, (int)heads, (int)head_dim, theta, (int)first,
                                        S(stream)));
}

static int append_common(void* stream, const float* src, size_t src_len, size_t src_off, void* dst, size_t dst_len,
                         int f16, size_t n, size_t kv, size_t hd, size_t cap, size_t past, int tr) {
    if (sadd(past, n) > cap) return overrun_cache(sadd(past, n), cap);
    if (f16 && cap % 2 != 0) return odd_cap(cap);
    if (int r = over_int(cap, kv, hd)) return r;
    const size_t total = smul(n, kv, hd);
    if (sadd(src_off, total) > src_len) return overrun_slice(sadd(src_off, total), src_len);
    if (smul(kv, cap, hd) > dst_len) return overrun_slice(smul(kv, cap, hd), dst_len);
    if (total == 0) return ok();
    if (!src || !dst) return invalid("a buffer");
    return launched("cache_append", launch_append(src, (long)src_off, dst, f16, tr, (int)n, (int)kv, (int)hd,
                                                  (int)cap, (int)past, S(stream)));
}

int llmtie_cache_append(void* stream, const float* src, size_t src_len, size_t src_off, float* dst, size_t dst_len,
                        size_t n, size_t kv_heads, size_t head_dim, size_t cap, size_t past, int transposed) {
    return append_common(stream, src, src_len, src_off, dst, dst_len, 0, n, kv_heads, head_dim, cap, past, transposed);
}

int llmtie_cache_append_f16(void* stream, const float* src, size_t src_len, size_t src_off, uint16_t* dst,
                            size_t dst_len, size_t n, size_t kv_heads, size_t head_dim, size_t cap, size_t past,
                            int transposed) {
    return append_common(stream, src, src_len, src_off, dst, dst_len, 1, n, kv_heads, head_dim, cap, past, transposed);
}

int llmtie_rope_cache_f16(void* stream, float* q, size_t q_len, size_t q_off, const float* k, size_t k_len,
                          size_t k_off, const float* v, size_t v_len, size_t v_off, const float* freq_div,
                          size_t heads, size_t kv_heads, size_t head_dim, float theta, size_t pos, uint16_t* kc,
                          uint16_t* vc, size_t cache_len, size_t cap) {
    if (pos >= cap) return overrun_cache(sadd(pos, 1), cap);
    if (cap % 2 != 0) return odd_cap(cap);
    if (head_dim % 2 != 0) return fail(LLMTIE_ODD_HEAD_DIM, head_dim, 0, 0, 0, "a rotary head of odd width %zu", head_dim);
    if (int r2 = over_int(cap, heads, head_dim)) return r2;
    if (sadd(q_off, heads * head_dim) > q_len) return overrun_slice(sadd(q_off, heads * head_dim), q_len);
    if (sadd(k_off, kv_heads * head_dim) > k_len) return overrun_slice(sadd(k_off, kv_heads * head_dim), k_len);
    if (sadd(v_off, kv_heads * head_dim) > v_len) return overrun_slice(sadd(v_off, kv_heads * head_dim), v_len);
    if (cache_len < smul(cap, kv_heads, head_dim)) return overrun_slice(smul(cap, kv_heads, head_dim), cache_len);
    if (!q || !k || !v || !kc || !vc) return invalid("a buffer");
    return launched("rope_cache_f16",
                    launch_rope_cache_f16(q, (long)q_off, k, (long)k_off, v, (long)v_off, freq_div, (int)heads,
                                          (int)kv_heads, (int)head_dim, theta, (int)pos, kc, vc, (int)cap, S(stream)));
}

static int grow_common(void* stream, const void* src, size_t src_len, void* dst, size_t dst_len, int esz, size_t kv,
                       size_t hd, size_t cap, size_t new_cap, size_t live, int tr) {
    if (live > cap || new_cap < cap) return overrun_cache(std::max(live, cap), std::min(new_cap, cap));
    size_t rows, len, ss, ds;
    if (!tr) {
        rows = kv;
        len = live * hd;
        ss = cap * hd;
        ds = new_cap * hd;
    } else {
        rows = kv * hd;
        len = live;
        ss = cap;
        ds = new_cap;
    }
    if (int r = over_int(rows, ss, ds)) return r;
    if (smul(rows, ss) > src_len) return overrun_slice(smul(rows, ss), src_len);
    if (smul(rows, ds) > dst_len) return overrun_slice(smul(rows, ds), dst_len);
    if (rows * len == 0) return ok();
    if (!src || !dst) return invalid("a buffer");
    return launched("cache_grow", launch_grow(src, dst, esz, (int)rows, (int)len, (int)ss, (int)ds, S(stream)));
}

int llmtie_cache_grow(void* stream, const float* src, size_t src_len, float* dst, size_t dst_len, size_t kv_heads,
                      size_t head_dim, size_t cap, size_t new_cap, size_t live, int transposed) {
    return grow_common(stream, src, src_len, dst, dst_len, 4, kv_heads, head_dim, cap, new_cap, live, transposed);
}

int llmtie_cache_grow_f16(void* stream, const uint16_t* src, size_t src_len, uint16_t* dst, size_t dst_len,
                          size_t kv_heads, size_t head_dim, size_t cap, size_t new_cap, size_t live,
                          int transposed) {
    return grow_common(stream, src, src_len, dst, dst_len, 2, kv_heads, head_dim, cap, new_cap, live, transposed);
}

static int q8_cache_checks(size_t hd, size_t heads, size_t kv, size_t cap, size_t slots, size_t slot,
                           size_t cache_len) {
    if (!(hd == 64 || hd == 128)) return unsupported(hd, heads, kv);
    if (slot >= slots) return overrun_slice(sadd(slot, 1), slots);
    if (int r = over_int(cap, slots, kv)) return r;
    const size_t need = llmtie_q8_cache_bytes(slots, kv, hd, cap);
    if (cache_len < need) return overrun_slice(need, cache_len);
    return LLMTIE_OK;
}

size_t llmtie_q8_cache_bytes(size_t slots, size_t kv_heads, size_t head_dim, size_t cap) {
    if (cap > IMAX) return SIZE_MAX;
    return smul(smul(slots, kv_heads), (size_t)tiled_nblk((int)cap), (size_t)tq8_block_bytes((int)head_dim));
}

size_t llmtie_t16_cache_len(size_t kv_heads, size_t head_dim, size_t cap) {
    if (cap > IMAX) return SIZE_MAX;
    return smul(smul(kv_heads, (size_t)tiled_nblk((int)cap)), 64, head_dim);
}

int llmtie_kv_q8_append(void* stream, const float* k, size_t k_len, size_t k_off, const float* v, size_t v_len,
                        size_t v_off, int8_t* cache, size_t cache_len, size_t slots, size_t slot, size_t n,
                        size_t kv_heads, size_t head_dim, size_t cap, size_t past) {
    int r = q8_cache_checks(head_dim, kv_heads, kv_heads, cap, slots, slot, cache_len);
    if (r != LLMTIE_OK) return r;
    if (sadd(past, n) > cap) return overrun_cache(sadd(past, n), cap);
    const size_t total = smul(n, kv_heads, head_dim);
    if (sadd(k_off, total) > k_len) return overrun_slice(sadd(k_off, total), k_len);
    if (sadd(v_off, total) > v_len) return overrun_slice(sadd(v_off, total), v_len);
    if (total == 0) return ok();
    if (!k || !v || !cache) return invalid("a buffer");
    return launched("kv_q8_append", launch_append_q8(k, (long)k_off, v, (long)v_off, reinterpret_cast<char*>(cache),
                                                     (int)slot, (int)n, (int)kv_heads, (int)head_dim, (int)cap,
                                                     (int)past, S(stream)));
}

int llmtie_rope_cache_q8(void* stream, float* q, size_t q_len, size_t q_off, const float* k, size_t k_len,
                         size_t k_off, const float* v, size_t v_len, size_t v_off, const float* freq_div,
                         size_t heads, size_t kv_heads, size_t head_dim, float theta, size_t pos, int8_t* cache,
                         size_t cache_len, size_t slots, size_t slot, size_t cap) {
    int r = q8_cache_checks(head_dim, heads, kv_heads, cap, slots, slot, cache_len);
    if (r != LLMTIE_OK) return r;
    if (pos >= cap) return overrun_cache(sadd(pos, 1), cap);
    if (int r2 = over_int(cap, heads, head_dim)) return r2;
    if (sadd(q_off, heads * head_dim) > q_len) return overrun_slice(sadd(q_off, heads * head_dim), q_len);
    if (sadd(k_off, kv_heads * head_dim) > k_len) return overrun_slice(sadd(k_off, kv_heads * head_dim), k_len);
    if (sadd(v_off, kv_heads * head_dim) > v_len) return overrun_slice(sadd(v_off, kv_heads * head_dim), v_len);
    if (!q || !k || !v || !cache) return invalid("a buffer");
    return launched("rope_cache_q8", launch_rope_cache_q8(q, (long)q_off, k, (long)k_off, v, (long)v_off, freq_div,
                                                          (int)heads, (int)kv_heads, (int)head_dim, theta, (int)pos,
                                                          reinterpret_cast<char*>(cache), (int)slot, (int)cap,
                                                          S(stream)));
}

// ------------------------------------------------------------ tiled f16

static int t16_checks(size_t hd, size_t heads, size_t kv, size_t cap, size_t cache_len) {
    if (!(hd == 64 || hd == 128) || kv == 0) return unsupported(hd, heads, kv);
    if (int r = over_int(cap, heads, kv)) return r;
    const size_t need = llmtie_t16_cache_len(kv, hd, cap);
    if (cache_len < need) return overrun_slice(need, cache_len);
    return LLMTIE_OK;
}

int llmtie_t16_append(void* stream, const float* src, size_t src_len, size_t src_off, uint16_t* cache,
                      size_t cache_len, size_t n, size_t kv_heads, size_t head_dim, size_t cap, size_t past,
                      int value) {
    int r = t16_checks(head_dim, kv_heads, kv_heads, cap, cache_len);
    if (r != LLMTIE_OK) return r;
    if (sadd(past, n) > cap) return overrun_cache(sadd(past, n), cap);
    const size_t total = smul(n, kv_heads, head_dim);
    if (sadd(src_off, total) > src_len) return overrun_slice(sadd(src_off, total), src_len);
    if (total == 0) return ok();
    if (!src || !cache) return invalid("a buffer");
    return launched("t16_append", launch_append_t16(src, (long)src_off, cache, (int)n, (int)kv_heads, (int)head_dim,
                                                    (int)cap, (int)past, value ? 1 : 0, S(stream)));
}

int llmtie_t16_rope_cache(void* stream, float* q, size_t q_len, size_t q_off, const float* k, size_t k_len,
                          size_t k_off, const float* v, size_t v_len, size_t v_off, const float* freq_div,
                          size_t heads, size_t kv_heads, size_t head_dim, float theta, size_t pos, uint16_t* cache,
                          size_t cache_len, size_t cap) {
    int r = t16_checks(head_dim, heads, kv_heads, cap, cache_len);
    if (r != LLMTIE_OK) return r;
    if (pos >= cap) return overrun_cache(sadd(pos, 1), cap);
    if (int r2 = over_int(cap, heads, head_dim)) return r2;
    if (sadd(q_off, heads * head_dim) > q_len) return overrun_slice(sadd(q_off, heads * head_dim), q_len);
    if (sadd(k_off, kv_heads * head_dim) > k_len) return overrun_slice(sadd(k_off, kv_heads * head_dim), k_len);
    if (sadd(v_off, kv_heads * head_dim) > v_len) return overrun_slice(sadd(v_off, kv_heads * head_dim), v_len);
    if (!q || !k || !v || !cache) return invalid("a buffer");
    return launched("t16_rope_cache",
                    launch_rope_cache_t16(q, (long)q_off, k, (long)k_off, v, (long)v_off, freq_div, (int)heads,
                                          (int)kv_heads, (int)head_dim, theta, (int)pos, cache, (int)cap, S(stream)));
}

int llmtie_t16_grow(void* stream, const uint16_t* src, size_t src_len, uint16_t* dst, size_t dst_len,
                    size_t kv_heads, size_t head_dim, size_t cap, size_t new_cap, size_t live) {
    if (live > cap || new_cap < cap) return overrun_cache(std::max(live, cap), std::min(new_cap, cap));
    int r = t16_checks(head_dim, kv_heads, kv_heads, cap, src_len);
    if (r != LLMTIE_OK) return r;
    r = t16_checks(head_dim, kv_heads, kv_heads, new_cap, dst_len);
    if (r != LLMTIE_OK) return r;
    const size_t bl = 64 * head_dim;  // halves per block
    const size_t rows = kv_heads, len = (size_t)tiled_nblk((int)live) * bl;
    if (rows * len == 0) return ok();
    if (!src || !dst) return invalid("a buffer");
    return launched("t16_grow", launch_grow(src, dst, 2, (int)rows, (int)len, (int)(tiled_nblk((int)cap) * bl),
                                            (int)(tiled_nblk((int)new_cap) * bl), S(stream)));
}

int llmtie_t16_from_ref(void* stream, const uint16_t* k, size_t k_len, const uint16_t* v, size_t v_len,
                        size_t kv_heads, size_t head_dim, size_t cap, size_t live, uint16_t* cache,
                        size_t cache_len) {
    int r = t16_checks(head_dim, kv_heads, kv_heads, cap, cache_len);
    if (r != LLMTIE_OK) return r;
    if (live > cap) return overrun_cache(live, cap);
    const size_t need = smul(kv_heads, cap, head_dim);
    if (k_len < need || v_len < need) return overrun_slice(need, std::min(k_len, v_len));
    if (live == 0) return ok();
    if (!k || !v || !cache) return invalid("a buffer");
    return launched("t16_from_ref", launch_ref_to_t16(k, v, cache, (int)kv_heads, (int)head_dim, (int)cap, (int)live,
                                                      (int)cap, S(stream)));
}

int llmtie_attn_decode_t16(void* stream, const float* q, size_t q_len, const uint16_t* cache, size_t cache_len,
                           size_t heads, size_t kv_heads, size_t head_dim, size_t tk, size_t cap, float scale,
                           int scale_q, llmtie_decode_scratch* scratch, float* out, size_t out_len) {
    return decode_common(stream, KV_T16, q, q_len, 0, cache, cache_len, nullptr, 0, heads, kv_heads, head_dim, tk,
                         cap, scale, scale_q, scratch, out, out_len, 0, nullptr, 0, 0, false);
}

int llmtie_attn_decode_t16_q_row(void* stream, const float* q, size_t q_len, size_t q_off, const uint16_t* cache,
                                 size_t cache_len, size_t heads, size_t kv_heads, size_t head_dim, size_t tk,
                                 size_t cap, float scale, int scale_q, llmtie_decode_scratch* scratch, float* out,
                                 size_t out_len, int8_t* twin, size_t twin_rows, size_t twin_k, size_t row) {
    return decode_common(stream, KV_T16, q, q_len, q_off, cache, cache_len, nullptr, 0, heads, kv_heads, head_dim,
                         tk, cap, scale, scale_q, scratch, out, out_len, smul(row, heads, head_dim), twin, twin_rows,
                         twin_k, twin != nullptr);
}

int llmtie_flash_attn_t16(void* stream, const float* q, size_t q_len, const uint16_t* cache, size_t cache_len,
                          float* out, size_t out_len, size_t tq, size_t past, size_t heads, size_t kv_heads,
                          size_t head_dim, size_t cap, float scale, int causal) {
    int r = t16_checks(head_dim, heads, kv_heads, cap, cache_len);
    if (r != LLMTIE_OK) return r;
    // The tiled cache holds both areas in one buffer; the length checks of the
    // shared path are satisfied by passing the whole-cache extent for both.
    const size_t ext = smul(kv_heads, cap, head_dim);
    return prefill_common(stream, PF_T16, q, q_len, cache, ext, cache, ext, out, out_len, tq, past, heads, kv_heads,
                          head_dim, cap, scale, causal);
}

}  // extern "C"
