// Weight quantisation on the device: Weight::quantize's q8 and q4 branches
// (crates/llm/src/quant.rs:209-281) and this build's Q4_K packing of GGML's
// block_q4_K (layout gpu/src/mpp.rs:241-282).
//
// Load-time work, one thread per 32-block (q8/q4) or per 256-weight
// super-block (Q4_K).  Every step is the reference's float operation in the
// reference's order (no contraction, correctly rounded divides), so the bytes
// equal the CPU quantiser's bit for bit.
#include "common.hpp"

namespace kh {
namespace {

__global__ void quantize_q8_kernel(const float *__restrict__ w, size_t nblocks, float *__restrict__ scales,
                                   int8_t *__restrict__ qs) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float *v = w + b * BLOCK;
    float amax = 0.0f;
    for (int k = 0; k < BLOCK; k++) amax = fmaxf(amax, fabsf(v[k]));
    float scale = amax / 127.0f;
    float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    scales[b] = scale;
    for (int k = 0; k < BLOCK; k++) {
        float t = v[k] * inv;
        t = roundf(t);
        t = fminf(fmaxf(t, -127.0f), 127.0f);
        qs[b * BLOCK + k] = (int8_t)(int)t;
    }
}

__global__ void quantize_q4_kernel(const float *__restrict__ w, size_t nblocks, float *__restrict__ scales,
                                   uint8_t *__restrict__ qs) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
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
        ta = fminf(fmaxf(ta, 0.0f), 15.0f);
        tb = fminf(fmaxf(tb, 0.0f), 15.0f);
        unsigned a = (unsigned)ta, c = (unsigned)tb;  // truncating, as `as u8`
        qs[b * (BLOCK / 2) + k] = (uint8_t)((a & 0x0f) | ((c & 0x0f) << 4));
    }
}

// Per 32-wide sub-block the range [min(w, 0), max(w)] in 15 steps; 6-bit
// scales and minimums under f16 super-block scales d and dmin.
__global__ void quantize_q4k_kernel(const float *__restrict__ w, size_t nsuper, uint8_t *__restrict__ out) {
    size_t s = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nsuper) return;
    const float *v = w + s * QK_K;
    uint8_t *blk = out + s * Q4K_BYTES;
    float scale[8], mins[8], smax = 0.0f, mmax = 0.0f;
    for (int j = 0; j < 8; j++) {
        float mn = 0.0f, mx = -INFINITY;
        for (int l = 0; l < 32; l++) {
            mn = fminf(mn, v[32 * j + l]);
            mx = fmaxf(mx, v[32 * j + l]);
        }
        if (mx < mn) mx = mn;
        scale[j] = (mx - mn) / 15.0f;
        mins[j] = -mn;
        smax = fmaxf(smax, scale[j]);
        mmax = fmaxf(mmax, mins[j]);
    }
    _Float16 dh = (_Float16)(smax / 63.0f), mh = (_Float16)(mmax / 63.0f);  // round to nearest even
    float d = (float)dh, dmin = (float)mh;
    uint8_t sc[8], mm[8];
    for (int j = 0; j < 8; j++) {
        float a = d > 0.0f ? roundf(scale[j] / d) : 0.0f;
        float b = dmin > 0.0f ? roundf(mins[j] / dmin) : 0.0f;
        sc[j] = (uint8_t)(a > 63.0f ? 63.0f : a);
        mm[j] = (uint8_t)(b > 63.0f ? 63.0f : b);
    }
    unsigned short dbits = __builtin_bit_cast(unsigned short, dh), mbits = __builtin_bit_cast(unsigned short, mh);
    blk[0] = dbits & 0xff;
    blk[1] = dbits >> 8;
    blk[2] = mbits & 0xff;
    blk[3] = mbits >> 8;
    uint8_t *q = blk + 4;
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((mm[j] & 63) | ((mm[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mm[j + 4] & 0xF) << 4));
    }
    uint8_t codes[128];
    for (int i = 0; i < 128; i++) codes[i] = 0;
    for (int j = 0; j < 8; j++) {
        float dl = d * (float)sc[j], ml = dmin * (float)mm[j];
        for (int l = 0; l < 32; l++) {
            float t = 0.0f;
            if (dl > 0.0f) {
                t = v[32 * j + l] + ml;
                t = t / dl;
                t = roundf(t);
                t = fminf(fmaxf(t, 0.0f), 15.0f);
            }
            codes[32 * (j / 2) + l] |= (uint8_t)((unsigned)t << (4 * (j & 1)));
        }
    }
    for (int i = 0; i < 128; i++) blk[16 + i] = codes[i];
}

}  // namespace

int launch_quantize(kh_ctx *ctx, const float *w, size_t rows, size_t cols, int precision, void *qs, float *scales) {
    const size_t n = rows * cols;
    dim3 block(128);
    if (precision == KH_Q8) {
        size_t nb = n / BLOCK;
        hipLaunchKernelGGL(quantize_q8_kernel, dim3((unsigned)((nb + 127) / 128)), block, 0, ctx->stream, w, nb, scales,
                           static_cast<int8_t *>(qs));
    } else if (precision == KH_Q4) {
        size_t nb = n / BLOCK;
        hipLaunchKernelGGL(quantize_q4_kernel, dim3((unsigned)((nb + 127) / 128)), block, 0, ctx->stream, w, nb, scales,
                           static_cast<uint8_t *>(qs));
    } else if (precision == KH_Q4K) {
        size_t ns = n / QK_K;
        hipLaunchKernelGGL(quantize_q4k_kernel, dim3((unsigned)((ns + 127) / 128)), block, 0, ctx->stream, w, ns,
                           static_cast<uint8_t *>(qs));
    } else {
        return fail(KH_EINVAL, "quantize: unknown precision");
    }
    KH_HIP(hipGetLastError());
    return KH_OK;
}

}  // namespace kh
