/*
 * CPU oracle for the attention hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's scalar CPU arithmetic, used by the
 * tests, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the
 * checker and the timed CPU baseline. Nothing in the product links or calls
 * it. Every function names the reference file:line it follows (paths relative
 * to the reference repository root).
 *
 * Compiled with -ffp-contract=off and no fast-math, so every f32 operation is
 * the single IEEE operation the reference's Rust performs.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------- binary16 */

/* IEEE binary16, round to nearest even: what `half::f16::from_f32` (half
 * 2.7.1, Cargo.lock:403-404) and `cvt.rn.f16.f32` (crates/llmtie-cuda/src/
 * kernels.rs:117-131) both compute. Bit-level, so it does not depend on the
 * host compiler's _Float16 support. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520: inf */
    if (ax < 0x38800000u) {                                     /* below the smallest normal half */
        if (ax < 0x33000000u) return (uint16_t)sign;            /* < 2^-25: rounds to zero */
        const uint32_t e = ax >> 23;                            /* 102 .. 112 */
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e;                         /* 14 .. 24 */
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24 */
            float f = (float)m * 5.9604644775390625e-8f;
            memcpy(&x, &f, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_f32_to_f16_n(const float* x, uint16_t* h, size_t n) {
    for (size_t i = 0; i < n; ++i) h[i] = orc_f32_to_f16(x[i]);
}
void orc_f16_to_f32_n(const uint16_t* h, float* x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = orc_f16_to_f32(h[i]);
}
static double h16(float x) { return (double)orc_f16_to_f32(orc_f32_to_f16(x)); }

/* ---------------------------------------------------------- generators */

/* The reference tests' deterministic spread, uniform on [-2, 6) (the doc
 * comment there says "roughly [-2, 2]"; the formula is what counts): xorshift64 with
 * shifts 13, 7, 17 seeded from salt * golden ratio | 1
 * (crates/llmtie-cuda/tests/kernels.rs:35-46). */
void orc_seq(float* out, size_t n, uint64_t salt) {
    uint64_t s = (salt * 0x9E3779B97F4A7C15ull) | 1ull;
    for (size_t i = 0; i < n; ++i) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        out[i] = ((float)(s >> 40) / 8388608.0f) * 4.0f - 2.0f;
    }
}

/* Counter-based N(0,1): splitmix64 of (seed, index) -> two uniforms ->
 * Box-Muller (cos branch), in double, rounded once to f32. Element i depends
 * only on (seed, i), so any slice of a tensor can be regenerated alone. */
static uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
void orc_normal(float* out, size_t n, uint64_t seed, uint64_t first) {
    for (size_t i = 0; i < n; ++i) {
        const uint64_t c = splitmix64(seed ^ 0xD1B54A32D192ED03ull) + 2ull * (first + i);
        const uint64_t a = splitmix64(c), b = splitmix64(c + 1);
        const double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0, 1] */
        const double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);         /* [0, 1) */
        out[i] = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
    }
}
/* Uniform integers in [lo, hi] from the same counter scheme. */
void orc_uniform_int(int32_t* out, size_t n, uint64_t seed, int32_t lo, int32_t hi) {
    const uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
    for (size_t i = 0; i < n; ++i) {
        const uint64_t a = splitmix64(splitmix64(seed ^ 0x5851F42D4C957F2Dull) + i);
        out[i] = (int32_t)((int64_t)lo + (int64_t)(a % span));
    }
}

/* --------------------------------------------------------------- RoPE */

/* crates/llmtie-dsp/src/rope.rs:83-126 (`rope_scaled`): halves pairing (i with
 * i + hd/2), inv = theta^(-2i/hd) in f32 (divided by freq_div[i] when given),
 * angle = (first + p) * inv in f32, f32 sin/cos. In place over [t, heads*hd]. */
void orc_rope(float* x, int t, int heads, int hd, float theta, int first, const float* freq_div) {
    const int half = hd / 2;
    for (int p = 0; p < t; ++p)
        for (int h = 0; h < heads; ++h) {
            const size_t base = ((size_t)p * heads + h) * hd;
            for (int i = 0; i < half; ++i) {
                float inv = powf(theta, -2.0f * (float)i / (float)hd);
                if (freq_div) inv /= freq_div[i];
                const float angle = (float)(first + p) * inv;
                const float s = sinf(angle), c = cosf(angle);
                const float a = x[base + i], b = x[base + i + half];
                x[base + i] = a * c - b * s;
                x[base + i + half] = b * c + a * s;
            }
        }
}

/* ------------------------------------------------------- decode (f32) */

/* crates/llmtie-cuda/tests/kernels.rs:2733-2780 (`decode_attention_ref`): the
 * three-kernel decode chain on the CPU for one query row. k is [kv][cap][hd],
 * v is [kv][hd][cap], both already at the precision the device cache holds.
 * Query head qh reads kv head qh / group. f32 throughout, sums in key order. */
void orc_decode_ref(const float* q, const float* k, const float* v, int heads, int kv, int hd, int tk, int cap,
                    float scale, int scale_q, float* out) {
    const int group = heads / kv;
    float* s = (float*)malloc(sizeof(float) * (size_t)(tk > 0 ? tk : 1));
    for (int qh = 0; qh < heads; ++qh) {
        const int h = qh / group;
        const float* qr = q + (size_t)qh * hd;
        for (int t = 0; t < tk; ++t) {
            const float* kr = k + ((size_t)h * cap + t) * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot += scale_q ? qr[d] * scale * kr[d] : qr[d] * kr[d];
            s[t] = scale_q ? dot : dot * scale;
        }
        float m = -INFINITY;
        for (int t = 0; t < tk; ++t) m = fmaxf(m, s[t]);
        float l = 0.0f;
        for (int t = 0; t < tk; ++t) {
            s[t] = expf(s[t] - m);
            l += s[t];
        }
        for (int d = 0; d < hd; ++d) {
            const float* vr = v + ((size_t)h * hd + d) * cap;
            float acc = 0.0f;
            for (int t = 0; t < tk; ++t) acc += s[t] * vr[t];
            out[(size_t)qh * hd + d] = acc / l;
        }
    }
    free(s);
}

/* The exact value decode_ref approximates: the same computation in f64 on the
 * same (already cache-precision) operands. The reference's own f32 chain
 * differs from it by up to ~2e-5 of full scale at 8k keys (sequential f32
 * sums), so tests hold the kernel to the reference's 2e-5 bar against this,
 * and against the f32 chain to that bar plus the chain's own deviation. */
void orc_decode_f64(const float* q, const float* k, const float* v, int heads, int kv, int hd, int tk, int cap,
                    float scale, int scale_q, double* out) {
    const int group = heads / kv;
    double* s = (double*)malloc(sizeof(double) * (size_t)(tk > 0 ? tk : 1));
    for (int qh = 0; qh < heads; ++qh) {
        const int h = qh / group;
        const float* qr = q + (size_t)qh * hd;
        double m = -INFINITY;
        for (int t = 0; t < tk; ++t) {
            const float* kr = k + ((size_t)h * cap + t) * hd;
            double dot = 0.0;
            for (int d = 0; d < hd; ++d) dot += (double)qr[d] * (double)kr[d];
            s[t] = dot * (double)scale;
            if (s[t] > m) m = s[t];
        }
        double l = 0.0;
        for (int t = 0; t < tk; ++t) {
            s[t] = exp(s[t] - m);
            l += s[t];
        }
        for (int d = 0; d < hd; ++d) {
            const float* vr = v + ((size_t)h * hd + d) * cap;
            double acc = 0.0;
            for (int t = 0; t < tk; ++t) acc += s[t] * (double)vr[t];
            out[(size_t)qh * hd + d] = acc / l;
        }
    }
    free(s);
    (void)scale_q;
}

/* The same over an f16 cache held as bits (the device layout), converted on
 * the fly: the CPU baseline for the f16 decode configs. `threads` > 1 splits
 * query heads over OpenMP threads; the arithmetic per head is unchanged. */
void orc_decode_f16(const float* q, const uint16_t* k, const uint16_t* v, int heads, int kv, int hd, int tk, int cap,
                    float scale, int scale_q, float* out, int threads) {
    const int group = heads / kv;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
#endif
    for (int qh = 0; qh < heads; ++qh) {
        float* s = (float*)malloc(sizeof(float) * (size_t)(tk > 0 ? tk : 1));
        const int h = qh / group;
        const float* qr = q + (size_t)qh * hd;
        for (int t = 0; t < tk; ++t) {
            const uint16_t* kr = k + ((size_t)h * cap + t) * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) {
                const float kk = orc_f16_to_f32(kr[d]);
                dot += scale_q ? qr[d] * scale * kk : qr[d] * kk;
            }
            s[t] = scale_q ? dot : dot * scale;
        }
        float m = -INFINITY;
        for (int t = 0; t < tk; ++t) m = fmaxf(m, s[t]);
        float l = 0.0f;
        for (int t = 0; t < tk; ++t) {
            s[t] = expf(s[t] - m);
            l += s[t];
        }
        for (int d = 0; d < hd; ++d) {
            const uint16_t* vr = v + ((size_t)h * hd + d) * cap;
            float acc = 0.0f;
            for (int t = 0; t < tk; ++t) acc += s[t] * orc_f16_to_f32(vr[t]);
            out[(size_t)qh * hd + d] = acc / l;
        }
        free(s);
    }
    (void)threads;
}

/* -------------------------------------------------------------- Q8_0 */

/* crates/llmtie-gguf/src/dequant.rs:180-185: a block is an f16 scale d and 32
 * int8 codes; element j = f32(d) * code[j]. Here codes and scales are passed
 * as separate arrays, one scale per 32 consecutive codes. */
void orc_q8_0_dequant(const int8_t* codes, const uint16_t* scales, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(scales[i / 32]) * (float)codes[i];
}

/* ggml's quantize_row_q8_0_ref (the GGUF Q8_0 writer; not vendored in the
 * reference, which only reads Q8_0): per 32 values amax = max|x|,
 * d = amax / 127, id = d ? 1/d : 0, code = roundf(x * id) (half away from
 * zero), scale stored as f16(d). */
void orc_q8_0_quantize(const float* x, size_t n, int8_t* codes, uint16_t* scales) {
    for (size_t b = 0; b < n / 32; ++b) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[b * 32 + j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        scales[b] = orc_f32_to_f16(d);
        for (int j = 0; j < 32; ++j) codes[b * 32 + j] = (int8_t)roundf(x[b * 32 + j] * id);
    }
}

/* The decode context's int8 twin as the reference's device epilogue makes it
 * (crates/llmtie-cuda/src/kernels.rs:5755-5773, `ad_emit`): per 32 values
 * d = max|y| * (1/127) (the f32 constant), inv = d > 0 ? 1/d : 0,
 * code = round-half-even(y * inv). Scales as f32. */
void orc_twin_quantize(const float* y, size_t n, int8_t* codes, float* scales) {
    for (size_t b = 0; b < n / 32; ++b) {
        float mx = 0.0f;
        for (int j = 0; j < 32; ++j) mx = fmaxf(mx, fabsf(y[b * 32 + j]));
        const float d = mx * (1.0f / 127.0f);
        const float inv = d > 0.0f ? 1.0f / d : 0.0f;
        scales[b] = d;
        for (int j = 0; j < 32; ++j) codes[b * 32 + j] = (int8_t)(int)nearbyintf(y[b * 32 + j] * inv);
    }
}

/* Batched decode over the Q8_0 cache layout of include/llmtie_hip.h, via
 * dequantisation then the f32 decode reference above (the Q8_0 path has no
 * reference implementation; it is pinned by the dequant closed form plus the
 * f32 attention oracle). q, out: [nseq][heads*hd]. */
void orc_decode_q8_batch(const float* q, const int8_t* kc, const uint16_t* ks, const int8_t* vc, const uint16_t* vs,
                         const int32_t* tk, const int32_t* slot, int nseq, int heads, int kv, int hd, int cap,
                         float scale, int scale_q, float* out, int threads) {
    const int nb = hd / 32;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(dynamic)
#endif
    for (int s = 0; s < nseq; ++s) {
        const int t = tk[s];
        const size_t sl = (size_t)slot[s];
        float* k = (float*)malloc(sizeof(float) * (size_t)kv * cap * hd);
        float* v = (float*)malloc(sizeof(float) * (size_t)kv * hd * cap);
        for (int h = 0; h < kv; ++h) {
            const size_t kvh = sl * kv + h;
            for (int p = 0; p < t; ++p)
                for (int d = 0; d < hd; ++d) {
                    const float dk = orc_f16_to_f32(ks[(kvh * cap + p) * nb + d / 32]);
                    const float dv = orc_f16_to_f32(vs[(kvh * cap + p) * nb + d / 32]);
                    k[((size_t)h * cap + p) * hd + d] = dk * (float)kc[(kvh * cap + p) * hd + d];
                    v[((size_t)h * hd + d) * cap + p] = dv * (float)vc[(kvh * hd + d) * cap + p];
                }
        }
        orc_decode_ref(q + (size_t)s * heads * hd, k, v, heads, kv, hd, t, cap, scale, scale_q,
                       out + (size_t)s * heads * hd);
        free(k);
        free(v);
    }
    (void)threads;
}

/* ------------------------------------------------------------- prefill */

/* crates/llmtie-cuda/tests/kernels.rs:2290-2374 (`fused_attention_sized`): the
 * f64 reference of the fused prefill. Operands rounded to f16 (q times the
 * scale first when scale_q, as kernels.rs:3090-3105 does), scores and
 * context accumulated in f64, probabilities rounded to f16 into the value
 * product, the normaliser summed from the unrounded ones. Row r of tq sees
 * keys 0..past+r when causal, else all past+tq keys. k [kv][cap][hd] and v
 * [kv][hd][cap] as f32 values (rounded here). Writes want and, for the
 * reference's tolerance 2e-4 + 1e-2|want| + 1e-2*spread, the spread: the
 * probability-weighted mean |v - want| of the values a row averages.
 * q [tq][qs] with head h at column h*hd; want/spread [tq][heads*hd]. */
void orc_prefill_ref(const float* q, int qs, const float* k, const float* v, int tq, int past, int heads, int kv,
                     int hd, int cap, float scale, int causal, int scale_q, double* want, double* spread,
                     int threads) {
    const int group = heads / kv;
    const int tk = past + tq;
    const int dq = heads * hd;
    /* The operands rounded once: K as [kv][tk][hd], V as [kv][hd][tk]. */
    double* kr = (double*)malloc(sizeof(double) * (size_t)kv * tk * hd);
    double* vr = (double*)malloc(sizeof(double) * (size_t)kv * hd * tk);
    for (int h = 0; h < kv; ++h)
        for (int p = 0; p < tk; ++p)
            for (int d = 0; d < hd; ++d) {
                kr[((size_t)h * tk + p) * hd + d] = h16(k[((size_t)h * cap + p) * hd + d]);
                vr[((size_t)h * hd + d) * tk + p] = h16(v[((size_t)h * hd + d) * cap + p]);
            }
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(dynamic)
#endif
    for (int hr = 0; hr < heads * tq; ++hr) {
        const int h = hr / tq, r = hr % tq;
        const int kh = h / group;
        const int last = causal ? past + r : tk - 1;
        double* s = (double*)malloc(sizeof(double) * (size_t)tk);
        double* e = (double*)malloc(sizeof(double) * (size_t)tk);
        double* pr = (double*)malloc(sizeof(double) * (size_t)tk);
        double* qd = (double*)malloc(sizeof(double) * (size_t)hd);
        for (int d = 0; d < hd; ++d) {
            const float qv = q[(size_t)r * qs + (size_t)h * hd + d];
            qd[d] = scale_q ? h16(qv * scale) : h16(qv);
        }
        double m = -INFINITY;
        for (int p = 0; p <= last; ++p) {
            const double* kk = kr + ((size_t)kh * tk + p) * hd;
            double acc = 0.0;
            for (int d = 0; d < hd; ++d) acc += qd[d] * kk[d];
            s[p] = scale_q ? acc : acc * (double)scale;
            if (s[p] > m) m = s[p];
        }
        double l = 0.0;
        for (int p = 0; p <= last; ++p) {
            e[p] = exp(s[p] - m);
            l += e[p];
            pr[p] = h16((float)e[p]);
        }
        for (int d = 0; d < hd; ++d) {
            const double* vv = vr + ((size_t)kh * hd + d) * tk;
            double acc = 0.0;
            for (int p = 0; p <= last; ++p) acc += pr[p] * vv[p];
            const double w = acc / l;
            double sp = 0.0;
            for (int p = 0; p <= last; ++p) sp += (e[p] / l) * fabs(vv[p] - w);
            want[(size_t)r * dq + (size_t)h * hd + d] = w;
            spread[(size_t)r * dq + (size_t)h * hd + d] = sp;
        }
        free(s);
        free(e);
        free(pr);
        free(qd);
    }
    free(kr);
    free(vr);
    (void)threads;
}

/* The f32 CPU prefill of config 1: for every query row the decode
 * reference's arithmetic (kernels.rs:2733-2780 above; softmax as
 * crates/llmtie-dsp/src/activation.rs:24-38 `softmax_rows`) over the keys the
 * row may see. q, k, v, out are [t][heads*hd] rows (MHA or GQA), causal. */
void orc_prefill_f32(const float* q, const float* k, const float* v, int t, int heads, int kv, int hd, float scale,
                     int causal, float* out, int threads) {
    const int group = heads / kv;
    const int dq = heads * hd, dk = kv * hd;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(dynamic)
#endif
    for (int hr = 0; hr < heads * t; ++hr) {
        const int h = hr / t, r = hr % t;
        const int kh = h / group;
        const int n = causal ? r + 1 : t;
        float* s = (float*)malloc(sizeof(float) * (size_t)n);
        const float* qr = q + (size_t)r * dq + (size_t)h * hd;
        for (int p = 0; p < n; ++p) {
            const float* kr = k + (size_t)p * dk + (size_t)kh * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot += qr[d] * kr[d];
            s[p] = dot * scale;
        }
        float m = -INFINITY;
        for (int p = 0; p < n; ++p) m = fmaxf(m, s[p]);
        float l = 0.0f;
        for (int p = 0; p < n; ++p) {
            s[p] = expf(s[p] - m);
            l += s[p];
        }
        for (int p = 0; p < n; ++p) s[p] /= l;
        for (int d = 0; d < hd; ++d) {
            float acc = 0.0f;
            for (int p = 0; p < n; ++p) acc += s[p] * v[(size_t)p * dk + (size_t)kh * hd + d];
            out[(size_t)r * dq + (size_t)h * hd + d] = acc;
        }
        free(s);
    }
    (void)threads;
}

int orc_has_openmp(void) {
#ifdef _OPENMP
    return 1;
#else
    return 0;
#endif
}
