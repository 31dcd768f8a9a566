// Single-token GEMV for kvad's q8 / q4 layouts, GGML Q4_K blocks and f32
// weights, plus the activation quantiser they consume.
//
// Reference: Weight::matvec_bt / qrow (crates/llm/src/quant.rs:410-512),
// q4_row_dots (quant.rs:168-189), matvec_many (quant.rs:628-671),
// QActivation::new (quant.rs:1044-1066), tensor::matvec_bt (tensor.rs:56-79),
// Q4_K decoding (crates/gpu/src/mpp.rs:241-315).
//
// Shape of the kernel.  A wave64 owns R whole weight rows.  Each row is cut
// into 16-byte chunks (q8: half a 32-block; q4: one block; Q4_K: half of two
// sub-blocks' nibbles; f32: four weights) and lane l takes chunks l, l+64,
// l+128, ... of every row it owns, so one load instruction of the wave moves
// 1 KiB of contiguous weight bytes.  The integer block dots are v_dot4 on
// int8 lanes; where a 32-block spans two lanes the halves are joined with a
// lane swap, so the i32 per block is exact.  The scaled f32 terms are
// summed per lane in chunk order and then across the wave.
//
// Bit-exactness.  Block dots (pass 1) equal the reference's integers.  Each
// f32 term is computed with the reference's operation order (quant.rs:449:
// (ws * xs) * d), and this file is compiled with -ffp-contract=off so no
// product is fused.  The sum over blocks is a wave tree, not the reference's
// two alternating accumulators, so outputs agree to rounding (1e-5
// relative), not to the bit.  The per-lane order depends only on the chunk
// index, never on the unroll (CPL) or rows per wave (R), so a row computed
// in a matvec_many launch equals the same row computed alone, to the bit.
#include "common.hpp"

namespace kh {
namespace {

constexpr int WAVE = 64;
constexpr int WAVES_PER_BLOCK = 4;
constexpr int MAX_JOBS = 24;

struct JobTable {
    GemvJob j[MAX_JOBS];
    int n;
};

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ int4 ld16(const void *p) { return *reinterpret_cast<const int4 *>(p); }

__device__ __forceinline__ int byte_of(const int4 &v, int k) {
    int w = k < 4 ? v.x : k < 8 ? v.y : k < 12 ? v.z : v.w;
    return (w >> (8 * (k & 3))) & 0xff;
}

__device__ __forceinline__ float half_bits_to_float(unsigned short h) {
    _Float16 f = __builtin_bit_cast(_Float16, h);
    return (float)f;
}

// Chunks of 16 bytes per weight row.
__host__ __device__ inline int chunks_per_row(int prec, int cols) {
    switch (prec) {
        case KH_Q8: return cols / 16;
        case KH_Q4: return cols / 32;
        case KH_Q4K: return (cols / QK_K) * 8;
        default: return (cols + 3) / 4;
    }
}

// ---------------------------------------------------------------------------
// activation quantiser: 8 lanes per 32-block, 4 values each
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void qact_kernel(const float *__restrict__ x, size_t nblocks,
                                                  int8_t *__restrict__ qs, float *__restrict__ scales,
                                                  int32_t *__restrict__ sums) {
    size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t b = tid >> 3;
    int sub = threadIdx.x & 7;
    bool ok = b < nblocks;
    float4 v = ok ? reinterpret_cast<const float4 *>(x)[b * 8 + sub] : make_float4(0.f, 0.f, 0.f, 0.f);
    // amax (quant.rs:1052): max is exact, so the lane order does not matter
    float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    a = fmaxf(a, __shfl_xor(a, 1));
    a = fmaxf(a, __shfl_xor(a, 2));
    a = fmaxf(a, __shfl_xor(a, 4));
    float scale = a / 127.0f;
    float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    float e[4] = {v.x, v.y, v.z, v.w};
    int packed = 0, s = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float t = e[k] * inv;
        t = roundf(t);
        t = fminf(fmaxf(t, -127.0f), 127.0f);
        int q = (int)t;
        s += q;
        packed |= (q & 0xff) << (8 * k);
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if (ok) {
        reinterpret_cast<int *>(qs)[b * 8 + sub] = packed;
        if (sub == 0) {
            scales[b] = scale;
            sums[b] = s;
        }
    }
}

// ---------------------------------------------------------------------------
// the GEMV kernel family
// ---------------------------------------------------------------------------

template <int PREC, int CPL, int R>
__global__ __launch_bounds__(256) void gemv_kernel(JobTable tab) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    int ji = 0;
    while (ji + 1 < tab.n && wave >= tab.j[ji + 1].wave0) ji++;
    const GemvJob &job = tab.j[ji];
    const int rows = job.rows, cols = job.cols;
    const int r0 = (wave - job.wave0) * R;
    if (wave < job.wave0 || r0 >= rows) return;

    const int C = chunks_per_row(PREC, cols);
    const int nb = cols / BLOCK;
    const int nseg = (C + WAVE * CPL - 1) / (WAVE * CPL);

    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++) acc[i] = 0.0f;

    for (int seg = 0; seg < nseg; seg++) {
        const int gbase = seg * WAVE * CPL + lane;
        if constexpr (PREC == KH_Q8) {
            const int8_t *W = static_cast<const int8_t *>(job.w);
            int4 w[R][CPL];
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int t = 0; t < CPL; t++) {
                    int g = gbase + t * WAVE, r = r0 + i;
                    w[i][t] = (g < C && r < rows) ? ld16(W + (size_t)r * cols + (size_t)g * 16) : int4{0, 0, 0, 0};
                }
            int4 a[CPL];
            float as[CPL];
#pragma unroll
            for (int t = 0; t < CPL; t++) {
                int g = gbase + t * WAVE;
                a[t] = g < C ? ld16(job.xq + (size_t)g * 16) : int4{0, 0, 0, 0};
                as[t] = g < C ? job.xs[g >> 1] : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int r = r0 + i;
#pragma unroll
                for (int t = 0; t < CPL; t++) {
                    const int g = gbase + t * WAVE;
                    int d = dot4(w[i][t].x, a[t].x, 0);
                    d = dot4(w[i][t].y, a[t].y, d);
                    d = dot4(w[i][t].z, a[t].z, d);
                    d = dot4(w[i][t].w, a[t].w, d);
                    d += __shfl_xor(d, 1);  // the other half of the 32-block
                    if (!(lane & 1) && g < C && r < rows) {
                        const int b = g >> 1;
                        float s = job.ws[(size_t)r * nb + b] * as[t];
                        s = s * (float)d;
                        acc[i] += s;
                        if (job.dots) job.dots[(size_t)r * nb + b] = d;
                    }
                }
            }
        } else if constexpr (PREC == KH_Q4) {
            const uint8_t *W = static_cast<const uint8_t *>(job.w);
            int4 w[R][CPL];
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int t = 0; t < CPL; t++) {
                    int g = gbase + t * WAVE, r = r0 + i;
                    w[i][t] = (g < C && r < rows) ? ld16(W + (size_t)r * (cols / 2) + (size_t)g * 16)
                                                  : int4{0, 0, 0, 0};
                }
            int4 alo[CPL], ahi[CPL];
            float as[CPL];
            int asum[CPL];
#pragma unroll
            for (int t = 0; t < CPL; t++) {
                int g = gbase + t * WAVE;
                bool ok = g < C;
                alo[t] = ok ? ld16(job.xq + (size_t)g * 32) : int4{0, 0, 0, 0};
                ahi[t] = ok ? ld16(job.xq + (size_t)g * 32 + 16) : int4{0, 0, 0, 0};
                as[t] = ok ? job.xs[g] : 0.0f;
                asum[t] = ok ? job.xsum[g] : 0;
            }
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int r = r0 + i;
#pragma unroll
                for (int t = 0; t < CPL; t++) {
                    const int g = gbase + t * WAVE;
                    const int4 q = w[i][t];
                    int lo = dot4(q.x & 0x0f0f0f0f, alo[t].x, 0);
                    lo = dot4(q.y & 0x0f0f0f0f, alo[t].y, lo);
                    lo = dot4(q.z & 0x0f0f0f0f, alo[t].z, lo);
                    lo = dot4(q.w & 0x0f0f0f0f, alo[t].w, lo);
                    int hi = dot4((q.x >> 4) & 0x0f0f0f0f, ahi[t].x, 0);
                    hi = dot4((q.y >> 4) & 0x0f0f0f0f, ahi[t].y, hi);
                    hi = dot4((q.z >> 4) & 0x0f0f0f0f, ahi[t].z, hi);
                    hi = dot4((q.w >> 4) & 0x0f0f0f0f, ahi[t].w, hi);
                    const int d = lo + hi - 8 * asum[t];  // quant.rs:187
                    if (g < C && r < rows) {
                        float s = job.ws[(size_t)r * nb + g] * as[t];
                        s = s * (float)d;
                        acc[i] += s;
                        if (job.dots) job.dots[(size_t)r * nb + g] = d;
                    }
                }
            }
        } else if constexpr (PREC == KH_Q4K) {
            const uint8_t *W = static_cast<const uint8_t *>(job.w);
            const size_t row_bytes = (size_t)(cols / QK_K) * Q4K_BYTES;
            int4 w[R][CPL], hdr[R][CPL];
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int t = 0; t < CPL; t++) {
                    int g = gbase + t * WAVE, r = r0 + i;
                    bool ok = g < C && r < rows;
                    const uint8_t *blk = W + (size_t)r * row_bytes + (size_t)(g >> 3) * Q4K_BYTES;
                    w[i][t] = ok ? ld16(blk + 16 + 16 * (g & 7)) : int4{0, 0, 0, 0};
                    hdr[i][t] = ok ? ld16(blk) : int4{0, 0, 0, 0};
                }
            // lane's chunk g covers, for sub-blocks j0 = 2c (low nibbles) and
            // j1 = 2c+1 (high nibbles), positions 16*half .. 16*half+15
            int4 alo[CPL], ahi[CPL];
            float as[CPL];
            int asum[CPL];
#pragma unroll
            for (int t = 0; t < CPL; t++) {
                int g = gbase + t * WAVE;
                bool ok = g < C;
                int sb = g >> 3, c = (g & 7) >> 1, half = g & 1;
                int b0 = sb * 8 + 2 * c;          // global 32-block of j0
                int bown = b0 + half;             // the sub-block this lane finishes
                alo[t] = ok ? ld16(job.xq + (size_t)b0 * 32 + 16 * half) : int4{0, 0, 0, 0};
                ahi[t] = ok ? ld16(job.xq + (size_t)(b0 + 1) * 32 + 16 * half) : int4{0, 0, 0, 0};
                as[t] = ok ? job.xs[bown] : 0.0f;
                asum[t] = ok ? job.xsum[bown] : 0;
            }
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int r = r0 + i;
#pragma unroll
                for (int t = 0; t < CPL; t++) {
                    const int g = gbase + t * WAVE;
                    const int4 q = w[i][t];
                    int lo = dot4(q.x & 0x0f0f0f0f, alo[t].x, 0);
                    lo = dot4(q.y & 0x0f0f0f0f, alo[t].y, lo);
                    lo = dot4(q.z & 0x0f0f0f0f, alo[t].z, lo);
                    lo = dot4(q.w & 0x0f0f0f0f, alo[t].w, lo);
                    int hi = dot4((q.x >> 4) & 0x0f0f0f0f, ahi[t].x, 0);
                    hi = dot4((q.y >> 4) & 0x0f0f0f0f, ahi[t].y, hi);
                    hi = dot4((q.z >> 4) & 0x0f0f0f0f, ahi[t].z, hi);
                    hi = dot4((q.w >> 4) & 0x0f0f0f0f, ahi[t].w, hi);
                    lo += __shfl_xor(lo, 1);
                    hi += __shfl_xor(hi, 1);
                    const int half = g & 1;
                    const int j = 2 * ((g & 7) >> 1) + half;
                    const int d = half ? hi : lo;
                    // 6-bit scale and minimum of sub-block j (mpp.rs:276-282)
                    const int4 h = hdr[i][t];
                    int sc, mn;
                    if (j < 4) {
                        sc = byte_of(h, 4 + j) & 63;
                        mn = byte_of(h, 8 + j) & 63;
                    } else {
                        sc = (byte_of(h, 8 + j) & 0xf) | ((byte_of(h, j) >> 6) << 4);
                        mn = (byte_of(h, 8 + j) >> 4) | ((byte_of(h, 4 + j) >> 6) << 4);
                    }
                    const float dl = half_bits_to_float((unsigned short)(h.x & 0xffff)) * (float)sc;
                    const float ml = half_bits_to_float((unsigned short)((unsigned)h.x >> 16)) * (float)mn;
                    if (g < C && r < rows) {
                        float t1 = dl * (float)d;
                        float t2 = ml * (float)asum[t];
                        float s = t1 - t2;
                        s = as[t] * s;
                        acc[i] += s;
                        if (job.dots) job.dots[(size_t)r * nb + (g >> 3) * 8 + j] = d;
                    }
                }
            }
        } else {  // KH_F32: chunk = 4 consecutive weights
            const float *W = static_cast<const float *>(job.w);
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int r = r0 + i;
#pragma unroll
                for (int t = 0; t < CPL; t++) {
                    const int g = gbase + t * WAVE;
                    if (g < C && r < rows) {
                        const float *wr = W + (size_t)r * cols;
                        float s = 0.0f;
                        for (int k = 4 * g; k < 4 * g + 4 && k < cols; k++) s = fmaf(wr[k], job.xf[k], s);
                        acc[i] += s;
                    }
                }
            }
        }
    }

#pragma unroll
    for (int i = 0; i < R; i++) {
        float v = wave_sum(acc[i]);
        const int r = r0 + i;
        if (lane == 0 && r < rows) job.y[r] = job.bias ? v + job.bias[r] : v;
    }
}

template <int PREC>
int launch_prec(kh_ctx *ctx, JobTable &tab, int maxC) {
    int cpl = (maxC + WAVE - 1) / WAVE;
    if (cpl < 1) cpl = 1;
    if (cpl > 8) cpl = 8;
    static const int rows_for_cpl[9] = {8, 8, 4, 2, 2, 1, 1, 1, 1};
    const int R = rows_for_cpl[cpl];
    int waves = 0;
    for (int i = 0; i < tab.n; i++) {
        tab.j[i].wave0 = waves;
        waves += (tab.j[i].rows + R - 1) / R;
    }
    if (waves == 0) return KH_OK;
    dim3 grid((waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK), block(WAVE * WAVES_PER_BLOCK);
    switch (cpl) {
        case 1: hipLaunchKernelGGL((gemv_kernel<PREC, 1, 8>), grid, block, 0, ctx->stream, tab); break;
        case 2: hipLaunchKernelGGL((gemv_kernel<PREC, 2, 4>), grid, block, 0, ctx->stream, tab); break;
        case 3: hipLaunchKernelGGL((gemv_kernel<PREC, 3, 2>), grid, block, 0, ctx->stream, tab); break;
        case 4: hipLaunchKernelGGL((gemv_kernel<PREC, 4, 2>), grid, block, 0, ctx->stream, tab); break;
        case 5: hipLaunchKernelGGL((gemv_kernel<PREC, 5, 1>), grid, block, 0, ctx->stream, tab); break;
        case 6: hipLaunchKernelGGL((gemv_kernel<PREC, 6, 1>), grid, block, 0, ctx->stream, tab); break;
        case 7: hipLaunchKernelGGL((gemv_kernel<PREC, 7, 1>), grid, block, 0, ctx->stream, tab); break;
        default: hipLaunchKernelGGL((gemv_kernel<PREC, 8, 1>), grid, block, 0, ctx->stream, tab); break;
    }
    KH_HIP(hipGetLastError());
    return KH_OK;
}

// ---------------------------------------------------------------------------
// small kernels
// ---------------------------------------------------------------------------

__global__ void fill_kernel(float *p, size_t n, float value) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = value;
}

// Weight::row (quant.rs:374-402) and the Q4_K decoder (mpp.rs:304-315).
__global__ void dequant_row_kernel(int prec, const void *qs, const float *scales, size_t cols, size_t r,
                                   float *out) {
    size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= cols) return;
    const size_t nb = cols / BLOCK;
    if (prec == KH_Q8) {
        const int8_t *q = static_cast<const int8_t *>(qs) + r * cols;
        out[k] = (float)q[k] * scales[r * nb + k / BLOCK];
    } else if (prec == KH_Q4) {
        const uint8_t *q = static_cast<const uint8_t *>(qs) + r * cols / 2;
        size_t b = k / BLOCK, o = k % BLOCK;
        uint8_t byte = q[b * 16 + (o & 15)];
        int code = o < 16 ? (byte & 0x0f) : (byte >> 4);
        out[k] = (float)(code - 8) * scales[r * nb + b];
    } else if (prec == KH_Q4K) {
        const uint8_t *blk = static_cast<const uint8_t *>(qs) + (r * (cols / QK_K) + k / QK_K) * Q4K_BYTES;
        int p = (int)(k % QK_K), j = p / 32, c = p / 64, h = (p / 32) & 1, l = p % 32;
        const uint8_t *s = blk + 4;
        int sc, mn;
        if (j < 4) {
            sc = s[j] & 63;
            mn = s[j + 4] & 63;
        } else {
            sc = (s[j + 4] & 0xf) | ((s[j - 4] >> 6) << 4);
            mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        unsigned short d16 = (unsigned short)(blk[0] | (blk[1] << 8));
        unsigned short m16 = (unsigned short)(blk[2] | (blk[3] << 8));
        float dl = half_bits_to_float(d16) * (float)sc;
        float ml = half_bits_to_float(m16) * (float)mn;
        int q = (blk[16 + 32 * c + l] >> (4 * h)) & 0xf;
        float t = dl * (float)q;
        out[k] = t - ml;
    } else {
        out[k] = static_cast<const float *>(qs)[r * cols + k];
    }
}

}  // namespace

int launch_qact(kh_ctx *ctx, const float *x, size_t m, size_t k, const QAct &out) {
    size_t nblocks = m * k / BLOCK;
    if (nblocks == 0) return KH_OK;
    size_t threads = nblocks * 8;
    dim3 grid((unsigned)((threads + 255) / 256)), block(256);
    hipLaunchKernelGGL(qact_kernel, grid, block, 0, ctx->stream, x, nblocks, out.qs, out.scales, out.sums);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int launch_gemv(kh_ctx *ctx, int precision, const GemvJob *jobs, int njobs) {
    for (int base = 0; base < njobs; base += MAX_JOBS) {
        JobTable tab{};
        tab.n = njobs - base < MAX_JOBS ? njobs - base : MAX_JOBS;
        int maxC = 0;
        for (int i = 0; i < tab.n; i++) {
            tab.j[i] = jobs[base + i];
            int c = chunks_per_row(precision, tab.j[i].cols);
            maxC = c > maxC ? c : maxC;
        }
        int rc;
        switch (precision) {
            case KH_Q8: rc = launch_prec<KH_Q8>(ctx, tab, maxC); break;
            case KH_Q4: rc = launch_prec<KH_Q4>(ctx, tab, maxC); break;
            case KH_Q4K: rc = launch_prec<KH_Q4K>(ctx, tab, maxC); break;
            case KH_F32: rc = launch_prec<KH_F32>(ctx, tab, maxC); break;
            default: return fail(KH_EINVAL, "unknown precision");
        }
        if (rc != KH_OK) return rc;
    }
    return KH_OK;
}

int launch_fill(kh_ctx *ctx, float *p, size_t n, float value) {
    if (n == 0) return KH_OK;
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, p, n, value);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int launch_dequant_row(kh_ctx *ctx, const kh_weight *w, size_t r, float *out) {
    hipLaunchKernelGGL(dequant_row_kernel, dim3((unsigned)((w->cols + 255) / 256)), dim3(256), 0, ctx->stream,
                       w->precision, (const void *)w->qs, (const float *)w->scales, w->cols, r, out);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

}  // namespace kh
