/*
 * kvad_oracle.c -- CPU restatement of kvad's quantised matmul and decode
 * attention.  TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline);
 * the product never links it.
 *
 * Build: gcc -O3 -ffp-contract=off -fopenmp -fPIC -shared (oracle/Makefile).
 * -ffp-contract=off because the reference is Rust, which never contracts
 * a*b+c into an FMA (crates/llm/src/tensor.rs:136-150).  Row loops are split
 * into one contiguous chunk per thread, as quant.rs:50-53 does with rayon;
 * every row is computed independently, so the thread count never changes a
 * result bit.
 *
 * Parity status of each function is recorded in the test suite
 * (tests/test_oracle_*.py): each is pinned by the reference's own
 * known-answer tests where they exist and otherwise by closed forms and
 * brute force.
 */
#include "kvad_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define BLOCK KVO_BLOCK

/* ------------------------------------------------------------------------- */
/* nervus::rng::Rng  (crates/nervus/src/rng.rs:7-39)                          */
/* ------------------------------------------------------------------------- */

void kvo_rng_init(kvo_rng *r, uint64_t seed) {
    /* rng.rs:13-16: a zero state is a fixed point, so seed 0 is replaced. */
    r->state = seed == 0 ? 0x9E3779B97F4A7C15ull : seed;
}

uint64_t kvo_rng_next(kvo_rng *r) {
    /* rng.rs:18-25 */
    uint64_t x = r->state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    r->state = x;
    return x * 0x2545F4914F6CDD1Dull;
}

float kvo_rng_uniform(kvo_rng *r) {
    /* rng.rs:28-32: top 24 bits over 2^24 */
    return (float)(kvo_rng_next(r) >> 40) / (float)(1u << 24);
}

float kvo_rng_normal(kvo_rng *r) {
    /* rng.rs:35-39: Box-Muller in f32 */
    float u1 = fmaxf(kvo_rng_uniform(r), FLT_MIN);
    float u2 = kvo_rng_uniform(r);
    const float tau = 6.28318530717958647692f;
    float a = -2.0f * logf(u1);
    float b = tau * u2;
    return sqrtf(a) * cosf(b);
}

void kvo_fill_normal(uint64_t seed, float scale, float *out, size_t n) {
    kvo_rng r;
    kvo_rng_init(&r, seed);
    for (size_t i = 0; i < n; i++) out[i] = kvo_rng_normal(&r) * scale;
}

/* ------------------------------------------------------------------------- */
/* threads                                                                    */
/* ------------------------------------------------------------------------- */

static int g_threads = 0;

void kvo_set_threads(int n) { g_threads = n; }

int kvo_get_threads(void) {
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------- */
/* quantisation                                                               */
/* ------------------------------------------------------------------------- */

/* Rust's `f32::round` is half away from zero, as C roundf.  clamp then a
 * truncating `as i8` cast (quant.rs:226). */
static inline int8_t q8_of(float v, float inv) {
    float t = v * inv;
    t = roundf(t);
    if (t < -127.0f) t = -127.0f;
    if (t > 127.0f) t = 127.0f;
    return (int8_t)t;
}

/* One 32-block: amax, scale = amax/127, inv, codes (quant.rs:220-227). */
static inline float q8_block(const float *v, int8_t *q, int32_t *sum) {
    float amax = 0.0f;
    for (int k = 0; k < BLOCK; k++) amax = fmaxf(amax, fabsf(v[k]));
    float scale = amax / 127.0f;
    float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    int32_t s = 0;
    for (int k = 0; k < BLOCK; k++) {
        q[k] = q8_of(v[k], inv);
        s += q[k];
    }
    if (sum) *sum = s;
    return scale;
}

void kvo_quantize_q8(const float *w, size_t rows, size_t cols, float *scales, int8_t *qs) {
    /* quant.rs:218-230 */
    size_t nb = rows * cols / BLOCK;
#pragma omp parallel for schedule(static) num_threads(kvo_get_threads())
    for (size_t b = 0; b < nb; b++) scales[b] = q8_block(w + b * BLOCK, qs + b * BLOCK, NULL);
}

void kvo_quantize_q4(const float *w, size_t rows, size_t cols, float *scales, uint8_t *qs) {
    /* quant.rs:231-278 */
    size_t nb = rows * cols / BLOCK;
#pragma omp parallel for schedule(static) num_threads(kvo_get_threads())
    for (size_t b = 0; b < nb; b++) {
        const float *v = w + b * BLOCK;
        float extreme = 0.0f;
        for (int k = 0; k < BLOCK; k++)
            if (fabsf(v[k]) > fabsf(extreme)) extreme = v[k];
        float scale = extreme / -8.0f;
        float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
        scales[b] = scale;
        for (int k = 0; k < BLOCK / 2; k++) {
            float ta = v[k] * inv;
            ta = ta + 8.5f;
            float tb = v[k + BLOCK / 2] * inv;
            tb = tb + 8.5f;
            /* `.clamp(0.0, 15.0) as u8`: clamp, then truncate */
            ta = ta < 0.0f ? 0.0f : (ta > 15.0f ? 15.0f : ta);
            tb = tb < 0.0f ? 0.0f : (tb > 15.0f ? 15.0f : tb);
            uint8_t a = (uint8_t)ta, c = (uint8_t)tb;
            qs[b * (BLOCK / 2) + k] = (uint8_t)((a & 0x0f) | ((c & 0x0f) << 4));
        }
    }
}

void kvo_qact(const float *x, size_t n, int8_t *qs, float *scales, int32_t *sums) {
    /* QActivation::new, quant.rs:1044-1066 */
    for (size_t b = 0; b < n / BLOCK; b++)
        scales[b] = q8_block(x + b * BLOCK, qs + b * BLOCK, &sums[b]);
}

void kvo_qact_batch(const float *xs, size_t m, size_t n, int8_t *qs, float *scales, int32_t *sums) {
    /* QActBatch::new, quant.rs:693-714 (the same per-row scheme) */
    size_t nb = n / BLOCK;
    for (size_t i = 0; i < m; i++) kvo_qact(xs + i * n, n, qs + i * n, scales + i * nb, sums + i * nb);
}

/* ------------------------------------------------------------------------- */
/* f16 <-> f32 (IEEE 754 binary16, round to nearest even)                     */
/* ------------------------------------------------------------------------- */

uint16_t kvo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                                   /* below 2^-14: subnormal */
        float af;
        memcpy(&af, &a, 4);
        uint32_t m = (uint32_t)rintf(af * 16777216.0f); /* units of 2^-24, RNE */
        return (uint16_t)(sign | m);
    }
    uint32_t e = (a >> 23) - 127 + 15;
    uint32_t mant = a & 0x7fffffu;
    uint32_t h = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float kvo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        float f = (float)m * (1.0f / 16777216.0f);
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ------------------------------------------------------------------------- */
/* Q4_K                                                                       */
/* ------------------------------------------------------------------------- */

/* mpp.rs:276-282: sub-block j's 6-bit scale and minimum. */
void kvo_q4k_scale_min(const uint8_t *q, int j, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Build-defined quantiser (any valid packing will do: kernel parity is
 * measured on the packed bytes).  Per 32-wide sub-block: range [min(w,0),
 * max(w)] over 15 steps; 6-bit scales and minimums under f16 d and dmin. */
static void q4k_block(const float *w, uint8_t *blk) {
    float scale[8], mins[8], smax = 0.0f, mmax = 0.0f;
    for (int j = 0; j < 8; j++) {
        float mn = 0.0f, mx = -INFINITY;
        for (int l = 0; l < 32; l++) {
            mn = fminf(mn, w[32 * j + l]);
            mx = fmaxf(mx, w[32 * j + l]);
        }
        if (mx < mn) mx = mn;
        scale[j] = (mx - mn) / 15.0f;
        mins[j] = -mn;
        smax = fmaxf(smax, scale[j]);
        mmax = fmaxf(mmax, mins[j]);
    }
    uint16_t d16 = kvo_f32_to_f16(smax / 63.0f), m16 = kvo_f32_to_f16(mmax / 63.0f);
    float d = kvo_f16_to_f32(d16), dmin = kvo_f16_to_f32(m16);
    uint8_t sc[8], mm[8];
    for (int j = 0; j < 8; j++) {
        float a = d > 0.0f ? roundf(scale[j] / d) : 0.0f;
        float b = dmin > 0.0f ? roundf(mins[j] / dmin) : 0.0f;
        sc[j] = (uint8_t)(a > 63.0f ? 63.0f : a);
        mm[j] = (uint8_t)(b > 63.0f ? 63.0f : b);
    }
    memcpy(blk + 0, &d16, 2);
    memcpy(blk + 2, &m16, 2);
    uint8_t *s = blk + 4;
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((mm[j] & 63) | ((mm[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mm[j + 4] & 0xF) << 4));
    }
    uint8_t *qs = blk + 16;
    memset(qs, 0, 128);
    for (int j = 0; j < 8; j++) {
        float dl = d * (float)sc[j], ml = dmin * (float)mm[j];
        for (int l = 0; l < 32; l++) {
            float t = 0.0f;
            if (dl > 0.0f) {
                t = (w[32 * j + l] + ml) / dl;
                t = roundf(t);
                t = t < 0.0f ? 0.0f : (t > 15.0f ? 15.0f : t);
            }
            uint8_t q = (uint8_t)t;
            qs[32 * (j / 2) + l] |= (uint8_t)(q << (4 * (j & 1)));
        }
    }
}

void kvo_quantize_q4k(const float *w, size_t rows, size_t cols, uint8_t *blocks) {
    size_t n = rows * cols / KVO_QK_K;
#pragma omp parallel for schedule(static) num_threads(kvo_get_threads())
    for (size_t i = 0; i < n; i++) q4k_block(w + i * KVO_QK_K, blocks + i * KVO_Q4K_BYTES);
}

/* Sub-block j of a block: dl = f32(d)*sc, ml = f32(dmin)*m (mpp.rs:308-310). */
static inline void q4k_dlml(const uint8_t *blk, int j, float *dl, float *ml) {
    uint16_t d16, m16;
    memcpy(&d16, blk, 2);
    memcpy(&m16, blk + 2, 2);
    uint8_t sc, m;
    kvo_q4k_scale_min(blk + 4, j, &sc, &m);
    *dl = kvo_f16_to_f32(d16) * (float)sc;
    *ml = kvo_f16_to_f32(m16) * (float)m;
}

static inline int q4k_code(const uint8_t *blk, int p) {
    /* mpp.rs:306-313: c = p/64, h = (p/32)&1, l = p%32 */
    int c = p / 64, h = (p / 32) & 1, l = p % 32;
    return (blk[16 + 32 * c + l] >> (4 * h)) & 0xF;
}

/* ------------------------------------------------------------------------- */
/* dequantised rows                                                           */
/* ------------------------------------------------------------------------- */

void kvo_row_q8(const float *scales, const int8_t *qs, size_t cols, size_t r, float *out) {
    /* quant.rs:378-388: (f32)q * s */
    size_t base = r * cols / BLOCK;
    for (size_t k = 0; k < cols; k++) out[k] = (float)qs[r * cols + k] * scales[base + k / BLOCK];
}

void kvo_row_q4(const float *scales, const uint8_t *qs, size_t cols, size_t r, float *out) {
    /* quant.rs:389-400: (f32)(nibble - 8) * s, low nibble = first half of the block */
    size_t base = r * cols / BLOCK;
    const uint8_t *row = qs + r * cols / 2;
    for (size_t b = 0; b < cols / BLOCK; b++) {
        float s = scales[base + b];
        for (int k = 0; k < BLOCK / 2; k++) {
            uint8_t byte = row[b * (BLOCK / 2) + k];
            out[b * BLOCK + k] = (float)((int)(byte & 0x0f) - 8) * s;
            out[b * BLOCK + BLOCK / 2 + k] = (float)((int)(byte >> 4) - 8) * s;
        }
    }
}

void kvo_row_q4k(const uint8_t *blocks, size_t cols, size_t r, float *out) {
    /* mpp.rs:304-315: dl*q - ml, rounded twice */
    size_t nsb = cols / KVO_QK_K;
    for (size_t s = 0; s < nsb; s++) {
        const uint8_t *blk = blocks + (r * nsb + s) * KVO_Q4K_BYTES;
        for (int p = 0; p < KVO_QK_K; p++) {
            float dl, ml;
            q4k_dlml(blk, p / 32, &dl, &ml);
            float t = dl * (float)q4k_code(blk, p);
            out[s * KVO_QK_K + p] = t - ml;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* pass 1: integer block dots                                                 */
/* ------------------------------------------------------------------------- */

static inline void dots_q8_row(const int8_t *wrow, const int8_t *xq, size_t nb, int32_t *d) {
    /* quant.rs:427-434 */
    for (size_t b = 0; b < nb; b++) {
        int32_t s = 0;
        for (int k = 0; k < BLOCK; k++) s += (int32_t)wrow[b * BLOCK + k] * (int32_t)xq[b * BLOCK + k];
        d[b] = s;
    }
}

static inline void dots_q4_row(const uint8_t *wrow, const int8_t *xq, const int32_t *sums, size_t nb,
                               int32_t *d) {
    /* quant.rs:178-188 portable path: unsigned nibbles, bias taken off per block */
    for (size_t b = 0; b < nb; b++) {
        int32_t lo = 0, hi = 0;
        for (int k = 0; k < BLOCK / 2; k++) {
            uint8_t w = wrow[b * (BLOCK / 2) + k];
            lo += (int32_t)(w & 0x0f) * (int32_t)xq[b * BLOCK + k];
            hi += (int32_t)(w >> 4) * (int32_t)xq[b * BLOCK + BLOCK / 2 + k];
        }
        d[b] = lo + hi - 8 * sums[b];
    }
}

static inline void dots_q4k_row(const uint8_t *row, const int8_t *xq, size_t nsb, int32_t *d) {
    for (size_t s = 0; s < nsb; s++) {
        const uint8_t *blk = row + s * KVO_Q4K_BYTES;
        for (int j = 0; j < 8; j++) {
            int32_t acc = 0;
            for (int l = 0; l < 32; l++)
                acc += q4k_code(blk, 32 * j + l) * (int32_t)xq[(s * 8 + j) * 32 + l];
            d[s * 8 + j] = acc;
        }
    }
}

void kvo_block_dots_q8(const int8_t *qs, size_t rows, size_t cols, const int8_t *xq, int32_t *dots) {
    size_t nb = cols / BLOCK;
#pragma omp parallel for schedule(static) num_threads(kvo_get_threads())
    for (size_t r = 0; r < rows; r++) dots_q8_row(qs + r * cols, xq, nb, dots + r * nb);
}

void kvo_block_dots_q4(const uint8_t *qs, size_t rows, size_t cols, const int8_t *xq,
                       const int32_t *xsums, int32_t *dots) {
    size_t nb = cols / BLOCK;
#pragma omp parallel for schedule(static) num_threads(kvo_get_threads())
    for (size_t r = 0; r < rows; r++) dots_q4_row(qs + r * cols / 2, xq, xsums, nb, dots + r * nb);
}

void kvo_block_dots_q4k(const uint8_t *blocks, size_t rows, size_t cols, const int8_t *xq, int32_t *dots) {
    size_t nb = cols / BLOCK, nsb = cols / KVO_QK_K;
#pragma omp parallel for schedule(static) num_threads(kvo_get_threads())
    for (size_t r = 0; r < rows; r++) dots_q4k_row(blocks + r * nsb * KVO_Q4K_BYTES, xq, nsb, dots + r * nb);
}

/* ------------------------------------------------------------------------- */
/* pass 2 and the GEMVs                                                       */
/* ------------------------------------------------------------------------- */

/* quant.rs:443-451: sums[b & 1] += ws * xs * d, two accumulators. */
static inline float pass2(const float *ws, const float *xs, const int32_t *d, size_t nb) {
    float s[2] = {0.0f, 0.0f};
    for (size_t b = 0; b < nb; b++) {
        float t = ws[b] * xs[b];
        t = t * (float)d[b];
        s[b & 1] = s[b & 1] + t;
    }
    return s[0] + s[1];
}

/* The Q4_K counterpart (build-defined): per sub-block
 * xs * (dl * dot - ml * sum), each product and the difference rounded once,
 * into the same two alternating accumulators. */
static inline float pass2_q4k(const uint8_t *row, const float *xs, const int32_t *xsums, const int32_t *d,
                              size_t nsb) {
    float s[2] = {0.0f, 0.0f};
    for (size_t sb = 0; sb < nsb; sb++) {
        const uint8_t *blk = row + sb * KVO_Q4K_BYTES;
        for (int j = 0; j < 8; j++) {
            size_t b = sb * 8 + j;
            float dl, ml;
            q4k_dlml(blk, j, &dl, &ml);
            float t1 = dl * (float)d[b];
            float t2 = ml * (float)xsums[b];
            float t = t1 - t2;
            t = xs[b] * t;
            s[b & 1] = s[b & 1] + t;
        }
    }
    return s[0] + s[1];
}

typedef struct {
    int8_t *qs;
    float *scales;
    int32_t *sums;
} qact_t;

static qact_t qact_alloc(const float *xs, size_t m, size_t n) {
    qact_t a;
    a.qs = (int8_t *)malloc(m * n);
    a.scales = (float *)malloc(sizeof(float) * m * n / BLOCK);
    a.sums = (int32_t *)malloc(sizeof(int32_t) * m * n / BLOCK);
    kvo_qact_batch(xs, m, n, a.qs, a.scales, a.sums);
    return a;
}

static void qact_free(qact_t *a) {
    free(a->qs);
    free(a->scales);
    free(a->sums);
}

static void add_bias(float *y, const float *bias, size_t n) {
    /* quant.rs:506-510 */
    if (bias)
        for (size_t i = 0; i < n; i++) y[i] = y[i] + bias[i];
}

void kvo_matvec_q8(const float *scales, const int8_t *qs, size_t rows, size_t cols, const float *x,
                   const float *bias, float *y) {
    /* quant.rs:487-503 */
    size_t nb = cols / BLOCK;
    qact_t a = qact_alloc(x, 1, cols);
#pragma omp parallel num_threads(kvo_get_threads())
    {
        int32_t *d = (int32_t *)malloc(sizeof(int32_t) * nb);
#pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++) {
            dots_q8_row(qs + r * cols, a.qs, nb, d);
            y[r] = pass2(scales + r * nb, a.scales, d, nb);
        }
        free(d);
    }
    qact_free(&a);
    add_bias(y, bias, rows);
}

void kvo_matvec_q4(const float *scales, const uint8_t *qs, size_t rows, size_t cols, const float *x,
                   const float *bias, float *y) {
    size_t nb = cols / BLOCK;
    qact_t a = qact_alloc(x, 1, cols);
#pragma omp parallel num_threads(kvo_get_threads())
    {
        int32_t *d = (int32_t *)malloc(sizeof(int32_t) * nb);
#pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++) {
            dots_q4_row(qs + r * cols / 2, a.qs, a.sums, nb, d);
            y[r] = pass2(scales + r * nb, a.scales, d, nb);
        }
        free(d);
    }
    qact_free(&a);
    add_bias(y, bias, rows);
}

void kvo_matvec_q4k(const uint8_t *blocks, size_t rows, size_t cols, const float *x, const float *bias,
                    float *y) {
    size_t nb = cols / BLOCK, nsb = cols / KVO_QK_K;
    qact_t a = qact_alloc(x, 1, cols);
#pragma omp parallel num_threads(kvo_get_threads())
    {
        int32_t *d = (int32_t *)malloc(sizeof(int32_t) * nb);
#pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++) {
            const uint8_t *row = blocks + r * nsb * KVO_Q4K_BYTES;
            dots_q4k_row(row, a.qs, nsb, d);
            y[r] = pass2_q4k(row, a.scales, a.sums, d, nsb);
        }
        free(d);
    }
    qact_free(&a);
    add_bias(y, bias, rows);
}

/* The same product as kvo_matvec_q4k, organised for the CPU baseline rather
 * than for reading against the reference: per super-block the eight (dl, ml)
 * pairs are decoded once, and each 32-byte group of codes is unpacked once
 * into its two sub-blocks' dots (contiguous int loops the compiler
 * vectorises).  The integers and every rounded step of pass 2 are those of
 * kvo_matvec_q4k, so the outputs are equal to the bit (tests/test_oracle.py). */
void kvo_matvec_q4k_fast(const uint8_t *blocks, size_t rows, size_t cols, const float *x, const float *bias,
                         float *y) {
    size_t nsb = cols / KVO_QK_K;
    qact_t a = qact_alloc(x, 1, cols);
#pragma omp parallel for schedule(static) num_threads(kvo_get_threads())
    for (size_t r = 0; r < rows; r++) {
        const uint8_t *row = blocks + r * nsb * KVO_Q4K_BYTES;
        float s[2] = {0.0f, 0.0f};
        for (size_t sb = 0; sb < nsb; sb++) {
            const uint8_t *blk = row + sb * KVO_Q4K_BYTES;
            const int8_t *xq = a.qs + sb * KVO_QK_K;
            uint16_t d16, m16;
            memcpy(&d16, blk, 2);
            memcpy(&m16, blk + 2, 2);
            const float d = kvo_f16_to_f32(d16), dmin = kvo_f16_to_f32(m16);
            int32_t dot[8];
            for (int c = 0; c < 4; c++) {
                const uint8_t *q = blk + 16 + 32 * c;
                const int8_t *xl = xq + 64 * c, *xh = xq + 64 * c + 32;
                int32_t lo = 0, hi = 0;
                for (int l = 0; l < 32; l++) {
                    lo += (int32_t)(q[l] & 0x0f) * (int32_t)xl[l];
                    hi += (int32_t)(q[l] >> 4) * (int32_t)xh[l];
                }
                dot[2 * c] = lo;
                dot[2 * c + 1] = hi;
            }
            for (int j = 0; j < 8; j++) {
                const size_t b = sb * 8 + j;
                uint8_t sc, m;
                kvo_q4k_scale_min(blk + 4, j, &sc, &m);
                const float dl = d * (float)sc, ml = dmin * (float)m;
                float t1 = dl * (float)dot[j];
                float t2 = ml * (float)a.sums[b];
                float t = t1 - t2;
                t = a.scales[b] * t;
                s[b & 1] = s[b & 1] + t;
            }
        }
        y[r] = s[0] + s[1];
    }
    qact_free(&a);
    add_bias(y, bias, rows);
}

static inline float matvec_f32_row(const float *row, const float *x, size_t cols) {
    /* tensor.rs:62-75: four lanes, pairwise combine, serial tail */
    float acc[4] = {0, 0, 0, 0};
    size_t n4 = cols / 4;
    for (size_t c = 0; c < n4; c++)
        for (int l = 0; l < 4; l++) {
            float p = row[c * 4 + l] * x[c * 4 + l];
            acc[l] = acc[l] + p;
        }
    float total = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    for (size_t i = cols - cols % 4; i < cols; i++) {
        float p = x[i] * row[i];
        total = total + p;
    }
    return total;
}

void kvo_matvec_f32(const float *w, size_t rows, size_t cols, const float *x, const float *bias, float *y) {
#pragma omp parallel for schedule(static) num_threads(kvo_get_threads())
    for (size_t r = 0; r < rows; r++) y[r] = matvec_f32_row(w + r * cols, x, cols);
    add_bias(y, bias, rows);
}

void kvo_matvec_dequant(int precision, const float *scales, const void *qs_, size_t rows, size_t cols,
                        const float *x, float *y) {
    /* quant.rs:522-589 */
    size_t nb = cols / BLOCK;
    float *xsums = NULL;
    if (precision == 2) {
        xsums = (float *)malloc(sizeof(float) * nb);
        for (size_t b = 0; b < nb; b++) {
            float s = 0.0f;
            for (int k = 0; k < BLOCK; k++) s = s + x[b * BLOCK + k];
            xsums[b] = s;
        }
    }
#pragma omp parallel for schedule(static) num_threads(kvo_get_threads())
    for (size_t r = 0; r < rows; r++) {
        float sums[4] = {0, 0, 0, 0};
        for (size_t b = 0; b < nb; b++) {
            float inner[4] = {0, 0, 0, 0};
            if (precision == 1) {
                const int8_t *wb = (const int8_t *)qs_ + r * cols + b * BLOCK;
                for (int c = 0; c < BLOCK / 4; c++)
                    for (int j = 0; j < 4; j++) {
                        float p = x[b * BLOCK + c * 4 + j] * (float)wb[c * 4 + j];
                        inner[j] = inner[j] + p;
                    }
                float sc = scales[r * nb + b];
                for (int j = 0; j < 4; j++) {
                    float p = sc * inner[j];
                    sums[j] = sums[j] + p;
                }
            } else {
                const uint8_t *wb = (const uint8_t *)qs_ + r * cols / 2 + b * (BLOCK / 2);
                for (int c = 0; c < BLOCK / 8; c++)
                    for (int j = 0; j < 4; j++) {
                        uint8_t q = wb[c * 4 + j];
                        float p = x[b * BLOCK + c * 4 + j] * (float)(q & 0x0f);
                        inner[j] = inner[j] + p;
                        p = x[b * BLOCK + BLOCK / 2 + c * 4 + j] * (float)(q >> 4);
                        inner[j] = inner[j] + p;
                    }
                float dot = (inner[0] + inner[1]) + (inner[2] + inner[3]);
                float e = 8.0f * xsums[b];
                dot = dot - e;
                float p = scales[r * nb + b] * dot;
                sums[0] = sums[0] + p;
            }
        }
        y[r] = (sums[0] + sums[1]) + (sums[2] + sums[3]);
    }
    free(xsums);
}

/* ------------------------------------------------------------------------- */
/* batched prefill                                                            */
/* ------------------------------------------------------------------------- */

/* finish (quant.rs:849-858): [rows, m] -> [m, rows], + bias (0.0 if none) */
static void finish(const float *out_t, size_t m, size_t rows, const float *bias, float *y) {
    for (size_t r = 0; r < rows; r++) {
        float add = bias ? bias[r] : 0.0f;
        for (size_t i = 0; i < m; i++) y[i * rows + r] = out_t[r * m + i] + add;
    }
}

void kvo_matmul_q8(const float *scales, const int8_t *qs, size_t rows, size_t cols, const float *xs,
                   size_t m, const float *bias, float *y) {
    if (m == 1) { /* quant.rs:767-769 */
        kvo_matvec_q8(scales, qs, rows, cols, xs, bias, y);
        return;
    }
    size_t nb = cols / BLOCK;
    qact_t a = qact_alloc(xs, m, cols);
    float *out_t = (float *)malloc(sizeof(float) * rows * m);
#pragma omp parallel num_threads(kvo_get_threads())
    {
        int32_t *d = (int32_t *)malloc(sizeof(int32_t) * nb);
#pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++)
            for (size_t i = 0; i < m; i++) { /* row_dot, quant.rs:865-907 */
                dots_q8_row(qs + r * cols, a.qs + i * cols, nb, d);
                out_t[r * m + i] = pass2(scales + r * nb, a.scales + i * nb, d, nb);
            }
        free(d);
    }
    finish(out_t, m, rows, bias, y);
    free(out_t);
    qact_free(&a);
}

void kvo_matmul_q4(const float *scales, const uint8_t *qs, size_t rows, size_t cols, const float *xs,
                   size_t m, const float *bias, float *y) {
    if (m == 1) {
        kvo_matvec_q4(scales, qs, rows, cols, xs, bias, y);
        return;
    }
    size_t nb = cols / BLOCK;
    qact_t a = qact_alloc(xs, m, cols);
    float *out_t = (float *)malloc(sizeof(float) * rows * m);
#pragma omp parallel num_threads(kvo_get_threads())
    {
        int32_t *d = (int32_t *)malloc(sizeof(int32_t) * nb);
#pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++)
            for (size_t i = 0; i < m; i++) {
                dots_q4_row(qs + r * cols / 2, a.qs + i * cols, a.sums + i * nb, nb, d);
                out_t[r * m + i] = pass2(scales + r * nb, a.scales + i * nb, d, nb);
            }
        free(d);
    }
    finish(out_t, m, rows, bias, y);
    free(out_t);
    qact_free(&a);
}

void kvo_matmul_q4k(const uint8_t *blocks, size_t rows, size_t cols, const float *xs, size_t m,
                    const float *bias, float *y) {
    if (m == 1) {
        kvo_matvec_q4k(blocks, rows, cols, xs, bias, y);
        return;
    }
    size_t nb = cols / BLOCK, nsb = cols / KVO_QK_K;
    qact_t a = qact_alloc(xs, m, cols);
    float *out_t = (float *)malloc(sizeof(float) * rows * m);
#pragma omp parallel num_threads(kvo_get_threads())
    {
        int32_t *d = (int32_t *)malloc(sizeof(int32_t) * nb);
#pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++) {
            const uint8_t *row = blocks + r * nsb * KVO_Q4K_BYTES;
            for (size_t i = 0; i < m; i++) {
                dots_q4k_row(row, a.qs + i * cols, nsb, d);
                out_t[r * m + i] = pass2_q4k(row, a.scales + i * nb, a.sums + i * nb, d, nsb);
            }
        }
        free(d);
    }
    finish(out_t, m, rows, bias, y);
    free(out_t);
    qact_free(&a);
}

float kvo_dot(const float *a, const float *b, size_t n) {
    /* tensor.rs:220-235: eight lanes, pairwise tree, serial tail */
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t n8 = n / 8;
    for (size_t c = 0; c < n8; c++)
        for (int l = 0; l < 8; l++) {
            float p = a[c * 8 + l] * b[c * 8 + l];
            acc[l] = acc[l] + p;
        }
    float total = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    for (size_t j = n - n % 8; j < n; j++) {
        float p = a[j] * b[j];
        total = total + p;
    }
    return total;
}

void kvo_gemm_f32(const float *xs, size_t m, const float *w, size_t rows, size_t k, float *out_t) {
    /* tensor.rs:102-186: chunks of RB = 4 rows; 4x4 micro-kernel over TB = 4
     * tokens when the chunk is whole; `dot` for short chunks and leftovers. */
    const size_t RB = 4, TB = 4;
    size_t nb = k / 4, tail = nb * 4;
    size_t nchunks = (rows + RB - 1) / RB;
#pragma omp parallel for schedule(static) num_threads(kvo_get_threads())
    for (size_t rb = 0; rb < nchunks; rb++) {
        size_t r0 = rb * RB;
        size_t rows_here = rows - r0 < RB ? rows - r0 : RB;
        float *dst = out_t + r0 * m;
        size_t t0 = 0;
        while (t0 + TB <= m) {
            if (rows_here == RB) {
                float acc[4][4][4];
                memset(acc, 0, sizeof(acc));
                for (size_t b = 0; b < nb; b++) {
                    size_t o = b * 4;
                    for (size_t r = 0; r < RB; r++)
                        for (size_t t = 0; t < TB; t++)
                            for (int l = 0; l < 4; l++) {
                                float p = w[(r0 + r) * k + o + l] * xs[(t0 + t) * k + o + l];
                                acc[r][t][l] = acc[r][t][l] + p;
                            }
                }
                for (size_t r = 0; r < RB; r++)
                    for (size_t t = 0; t < TB; t++) {
                        float *a = acc[r][t];
                        float total = (a[0] + a[1]) + (a[2] + a[3]);
                        for (size_t j = tail; j < k; j++) {
                            float p = w[(r0 + r) * k + j] * xs[(t0 + t) * k + j];
                            total = total + p;
                        }
                        dst[r * m + t0 + t] = total;
                    }
            } else {
                for (size_t r = 0; r < rows_here; r++)
                    for (size_t t = 0; t < TB; t++)
                        dst[r * m + t0 + t] = kvo_dot(w + (r0 + r) * k, xs + (t0 + t) * k, k);
            }
            t0 += TB;
        }
        while (t0 < m) {
            for (size_t r = 0; r < rows_here; r++) dst[r * m + t0] = kvo_dot(w + (r0 + r) * k, xs + t0 * k, k);
            t0 += 1;
        }
    }
}

void kvo_matmul_f32(const float *w, size_t rows, size_t cols, const float *xs, size_t m, const float *bias,
                    float *y) {
    if (m == 1) { /* Weight::matmul_bt: m == 1 -> matvec_bt -> tensor::matvec_bt */
        kvo_matvec_f32(w, rows, cols, xs, bias, y);
        return;
    }
    float *out_t = (float *)malloc(sizeof(float) * rows * m);
    kvo_gemm_f32(xs, m, w, rows, cols, out_t);
    finish(out_t, m, rows, bias, y);
    free(out_t);
}

/* ------------------------------------------------------------------------- */
/* small f32 pieces                                                           */
/* ------------------------------------------------------------------------- */

void kvo_softmax(float *x, size_t n) {
    /* tensor.rs:297-308 */
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = fmaxf(mx, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum = sum + x[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] = x[i] * inv;
}

void kvo_rms_norm(const float *x, const float *w, size_t n, float eps, float *out) {
    /* tensor.rs:329-333 */
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float p = x[i] * x[i];
        ss = ss + p;
    }
    float ms = ss / (float)n;
    float inv = 1.0f / sqrtf(ms + eps);
    for (size_t i = 0; i < n; i++) {
        float t = x[i] * inv;
        out[i] = t * w[i];
    }
}

void kvo_swiglu(float *gate, const float *up, size_t n) {
    /* tensor.rs:344-350 */
    for (size_t i = 0; i < n; i++) {
        float g = gate[i];
        float silu = g / (1.0f + expf(-g));
        gate[i] = silu * up[i];
    }
}

void kvo_rope_tables(size_t head_dim, size_t max_pos, float theta, float *cos_t, float *sin_t) {
    /* tensor.rs:390-407 */
    size_t half = head_dim / 2;
    for (size_t pos = 0; pos < max_pos; pos++)
        for (size_t i = 0; i < half; i++) {
            float e = (2.0f * (float)i) / (float)head_dim;
            float inv_freq = 1.0f / powf(theta, e);
            float angle = (float)pos * inv_freq;
            cos_t[pos * half + i] = cosf(angle);
            sin_t[pos * half + i] = sinf(angle);
        }
}

void kvo_rope_apply(const float *cos_t, const float *sin_t, size_t half, float *x, size_t pos) {
    /* tensor.rs:463-472: pairs i and i + half */
    size_t base = pos * half;
    for (size_t i = 0; i < half; i++) {
        float c = cos_t[base + i], s = sin_t[base + i];
        float a = x[i], b = x[i + half];
        float p1 = a * c, p2 = b * s;
        x[i] = p1 - p2;
        float p3 = b * c, p4 = a * s;
        x[i + half] = p3 + p4;
    }
}

void kvo_rope_apply_interleaved(const float *cos_t, const float *sin_t, size_t half, float *x, size_t pos) {
    /* tensor.rs:437-446: pairs 2i and 2i + 1 */
    size_t base = pos * half;
    for (size_t i = 0; i < half; i++) {
        float c = cos_t[base + i], s = sin_t[base + i];
        float a = x[2 * i], b = x[2 * i + 1];
        float p1 = a * c, p2 = b * s;
        x[2 * i] = p1 - p2;
        float p3 = b * c, p4 = a * s;
        x[2 * i + 1] = p3 + p4;
    }
}

/* ------------------------------------------------------------------------- */
/* attention                                                                  */
/* ------------------------------------------------------------------------- */

void kvo_attend(size_t n_head, size_t n_kv_head, size_t hd, const float *q, const float *k_cache,
                const float *v_cache, size_t n_positions, float *out) {
    /* model/mod.rs:769-819 */
    size_t kv_dim = n_kv_head * hd;
    size_t group = n_head / n_kv_head;
    float scale = 1.0f / sqrtf((float)hd);
    memset(out, 0, sizeof(float) * n_head * hd);
#pragma omp parallel num_threads(kvo_get_threads())
    {
        float *scores = (float *)malloc(sizeof(float) * (n_positions ? n_positions : 1));
#pragma omp for schedule(static)
        for (size_t head = 0; head < n_head; head++) {
            const float *qh = q + head * hd;
            size_t kv_off = (head / group) * hd;
            for (size_t t = 0; t < n_positions; t++) {
                float d = kvo_dot(qh, k_cache + t * kv_dim + kv_off, hd);
                scores[t] = d * scale;
            }
            kvo_softmax(scores, n_positions);
            float *slot = out + head * hd;
            for (size_t t = 0; t < n_positions; t++) {
                float w = scores[t];
                if (w < 1e-8f) continue; /* mod.rs:807 */
                const float *vh = v_cache + t * kv_dim + kv_off;
                for (size_t i = 0; i < hd; i++) {
                    float p = w * vh[i];
                    slot[i] = slot[i] + p;
                }
            }
        }
        free(scores);
    }
}

/* Latent attention, absorbed (model/deepseek.rs:553-591): head h scores
 * position t as (dot(q_lat_h, c_t) + dot(q_pe_h, pe_t)) * scale, softmax
 * over the positions, then averages the compressed rows c_t, skipping
 * weights below 1e-8.  The uk / uv projections around it are matvecs. */
void kvo_mla_attend(size_t n_head, size_t lat, size_t rope, const float *q_lat, const float *q_pe,
                    const float *c_cache, const float *pe_cache, size_t n_positions, float scale, float *out) {
    memset(out, 0, sizeof(float) * n_head * lat);
#pragma omp parallel num_threads(kvo_get_threads())
    {
        float *scores = (float *)malloc(sizeof(float) * (n_positions ? n_positions : 1));
#pragma omp for schedule(static)
        for (size_t h = 0; h < n_head; h++) {
            const float *ql = q_lat + h * lat, *qp = q_pe + h * rope;
            for (size_t t = 0; t < n_positions; t++) {
                float a = kvo_dot(ql, c_cache + t * lat, lat);
                float b = kvo_dot(qp, pe_cache + t * rope, rope);
                float d = a + b;
                scores[t] = d * scale;
            }
            kvo_softmax(scores, n_positions);
            float *acc = out + h * lat;
            for (size_t t = 0; t < n_positions; t++) {
                float w = scores[t];
                if (w < 1e-8f) continue;
                const float *c = c_cache + t * lat;
                for (size_t j = 0; j < lat; j++) {
                    float p = w * c[j];
                    acc[j] = acc[j] + p;
                }
            }
        }
        free(scores);
    }
}

/* ------------------------------------------------------------------------- */
/* router                                                                     */
/* ------------------------------------------------------------------------- */

/* f32::total_cmp as an integer key: the IEEE bits with the magnitude bits
 * flipped for negatives, so -0.0 < +0.0 and the order is total. */
static int32_t total_key(float f) {
    int32_t b;
    memcpy(&b, &f, sizeof b);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

int kvo_route(const float *logits, size_t n, size_t top_k, int scoring, int select, size_t n_group,
              size_t topk_group, int norm_topk, float scale, const float *bias, int32_t *experts,
              float *weights) {
    /* model/ffn.rs:256-309 */
    float *scores = (float *)malloc(sizeof(float) * n);
    float *choice = (float *)malloc(sizeof(float) * n);
    memcpy(scores, logits, sizeof(float) * n);
    if (scoring == 0) {
        kvo_softmax(scores, n);
    } else {
        for (size_t i = 0; i < n; i++) scores[i] = 1.0f / (1.0f + expf(-scores[i]));
    }
    memcpy(choice, scores, sizeof(float) * n);
    if (bias)
        for (size_t i = 0; i < n; i++) choice[i] = choice[i] + bias[i];
    if (select != 0 && n_group > 1) {
        /* mask_to_best_groups, ffn.rs:312-349; a stable sort by descending
         * strength, as Rust's sort_by with total_cmp */
        size_t per = n / n_group;
        float *strength = (float *)malloc(sizeof(float) * n_group);
        size_t *order = (size_t *)malloc(sizeof(size_t) * n_group);
        for (size_t g = 0; g < n_group; g++) {
            const float *grp = choice + g * per;
            if (select == 1) {
                float mx = -INFINITY;
                for (size_t i = 0; i < per; i++) mx = fmaxf(mx, grp[i]);
                strength[g] = mx;
            } else {
                float a = -INFINITY, b = -INFINITY;
                for (size_t i = 0; i < per; i++) {
                    float v = grp[i];
                    if (v > a) {
                        b = a;
                        a = v;
                    } else if (v > b) {
                        b = v;
                    }
                }
                strength[g] = a + b;
            }
            order[g] = g;
        }
        for (size_t i = 1; i < n_group; i++) { /* stable insertion sort, descending by total_cmp */
            size_t x = order[i];
            size_t j = i;
            while (j > 0 && total_key(strength[order[j - 1]]) < total_key(strength[x])) {
                order[j] = order[j - 1];
                j--;
            }
            order[j] = x;
        }
        size_t keep = topk_group < n_group ? topk_group : n_group;
        for (size_t o = keep; o < n_group; o++)
            for (size_t i = 0; i < per; i++) choice[order[o] * per + i] = -INFINITY;
        free(strength);
        free(order);
    }
    size_t k = top_k < n ? top_k : n;
    int got = 0;
    for (size_t pick = 0; pick < k; pick++) {
        size_t best = (size_t)-1;
        for (size_t i = 0; i < n; i++)
            if (choice[i] > -INFINITY && (best == (size_t)-1 || choice[i] > choice[best])) best = i;
        if (best == (size_t)-1) break;
        experts[got] = (int32_t)best;
        weights[got] = scores[best];
        got++;
        choice[best] = -INFINITY;
    }
    int normalised = norm_topk && top_k > 1;
    if (normalised) {
        float total = 0.0f;
        for (int i = 0; i < got; i++) total = total + weights[i];
        total = total + 1e-20f;
        for (int i = 0; i < got; i++) weights[i] = weights[i] / total;
    }
    int always_scale = select == 2;
    if (always_scale || !normalised)
        for (int i = 0; i < got; i++) weights[i] = weights[i] * scale;
    free(scores);
    free(choice);
    return got;
}

/* ------------------------------------------------------------------------- */
/* mixture of experts                                                         */
/* ------------------------------------------------------------------------- */

/* Ffn::run / Ffn::run_one (model/ffn.rs:370-388): gate and up, SwiGLU, down.
 * m == 1 goes through matvec, as matmul_bt does (quant.rs:767-769). */
static void ffn_q8(const float *xs, size_t m, size_t hidden, size_t inter, const float *gs, const int8_t *gq,
                   const float *us, const int8_t *uq, const float *ds, const int8_t *dq, float *y) {
    float *g = (float *)malloc(sizeof(float) * m * inter);
    float *u = (float *)malloc(sizeof(float) * m * inter);
    kvo_matmul_q8(gs, gq, inter, hidden, xs, m, NULL, g);
    kvo_matmul_q8(us, uq, inter, hidden, xs, m, NULL, u);
    kvo_swiglu(g, u, m * inter);
    kvo_matmul_q8(ds, dq, hidden, inter, g, m, NULL, y);
    free(g);
    free(u);
}

void kvo_moe_run_q8(const float *hs, size_t m, size_t hidden, size_t inter, size_t n_exp, size_t top_k,
                    int scoring, int select, size_t n_group, size_t topk_group, int norm_topk, float scale,
                    const float *bias, const float *r_s, const int8_t *r_q, const float *g_s, const int8_t *g_q,
                    const float *u_s, const int8_t *u_q, const float *d_s, const int8_t *d_q, size_t sh_inter,
                    const float *sg_s, const int8_t *sg_q, const float *su_s, const int8_t *su_q,
                    const float *sd_s, const int8_t *sd_q, float *out) {
    /* Moe::run (ffn.rs:615-708) with mix (:744-806) and decode_together
     * (:820-842).  Expert x's gate/up are rows [x*inter, (x+1)*inter) of
     * g/u, its down rows [x*hidden, (x+1)*hidden) of d; scales alike. */
    const size_t gsz = inter * hidden, gsb = gsz / KVO_BLOCK;
    float *logits = (float *)malloc(sizeof(float) * m * n_exp);
    kvo_matmul_q8(r_s, r_q, n_exp, hidden, hs, m, NULL, logits);
    int32_t *pe = (int32_t *)malloc(sizeof(int32_t) * m * (top_k ? top_k : 1));
    float *pw = (float *)malloc(sizeof(float) * m * (top_k ? top_k : 1));
    int *np = (int *)malloc(sizeof(int) * m);
    for (size_t i = 0; i < m; i++)
        np[i] = kvo_route(logits + i * n_exp, n_exp, top_k, scoring, select, n_group, topk_group, norm_topk, scale,
                          bias, pe + i * top_k, pw + i * top_k);
    /* the shared expert first: out starts as its output (ffn.rs:675-681, 775-785) */
    if (sh_inter)
        ffn_q8(hs, m, hidden, sh_inter, sg_s, sg_q, su_s, su_q, sd_s, sd_q, out);
    else
        memset(out, 0, sizeof(float) * m * hidden);
    /* then each chosen expert in index order, its tokens in token order */
    float *rows = (float *)malloc(sizeof(float) * m * hidden);
    float *y = (float *)malloc(sizeof(float) * m * hidden);
    size_t *tok = (size_t *)malloc(sizeof(size_t) * m);
    float *wt = (float *)malloc(sizeof(float) * m);
    for (size_t x = 0; x < n_exp; x++) {
        size_t cnt = 0;
        for (size_t i = 0; i < m; i++)
            for (int k = 0; k < np[i]; k++)
                if ((size_t)pe[i * top_k + k] == x) {
                    tok[cnt] = i;
                    wt[cnt] = pw[i * top_k + k];
                    memcpy(rows + cnt * hidden, hs + i * hidden, sizeof(float) * hidden);
                    cnt++;
                }
        if (!cnt) continue;
        ffn_q8(rows, cnt, hidden, inter, g_s + x * gsb, g_q + x * gsz, u_s + x * gsb, u_q + x * gsz,
               d_s + x * gsb, d_q + x * gsz, y);
        for (size_t j = 0; j < cnt; j++)
            for (size_t e = 0; e < hidden; e++) {
                float p = wt[j] * y[j * hidden + e];
                out[tok[j] * hidden + e] = out[tok[j] * hidden + e] + p;
            }
    }
    free(rows);
    free(y);
    free(tok);
    free(wt);
    free(logits);
    free(pe);
    free(pw);
    free(np);
}
