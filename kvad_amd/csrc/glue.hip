// The decode step's glue between the matmuls and the attention:
// tensor::rms_norm (crates/llm/src/tensor.rs:329-333), Rope::apply and
// apply_interleaved (tensor.rs:437-472), swiglu_inplace (tensor.rs:344-350)
// and softmax_inplace (tensor.rs:297-308), on device arrays.
//
// RoPE is bit-exact: it multiplies by the caller's own cos/sin tables (the
// reference hands them out for exactly this, Rope::tables, tensor.rs:377-387)
// with the reference's two products and one sum.  RMSNorm and softmax reduce
// with a fixed tree rather than the reference's serial sum, and SwiGLU and
// softmax use the device's exp, so those agree to rounding.
#include "common.hpp"

namespace kh {
namespace {

// Fixed-order sum over a 256-thread block; every thread gets the total.
__device__ float block_sum(float v, float *s_red) {
    const int tid = threadIdx.x;
    s_red[tid] = v;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) s_red[tid] = s_red[tid] + s_red[tid + w];
        __syncthreads();
    }
    const float r = s_red[0];
    __syncthreads();
    return r;
}

__device__ float block_max(float v, float *s_red) {
    const int tid = threadIdx.x;
    s_red[tid] = v;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) s_red[tid] = fmaxf(s_red[tid], s_red[tid + w]);
        __syncthreads();
    }
    const float r = s_red[0];
    __syncthreads();
    return r;
}

// One row per workgroup: mean of squares, inv = 1 / sqrt(ms + eps),
// out = (x * inv) * w.
__global__ __launch_bounds__(256) void rms_norm_kernel(const float *x, const float *w, int n, float eps, float *out) {
    __shared__ float s_red[256];
    const float *xr = x + (size_t)blockIdx.x * n;
    float *o = out + (size_t)blockIdx.x * n;
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = xr[i];
        const float sq = v * v;
        s = s + sq;
    }
    const float ms = block_sum(s, s_red) / (float)n;
    const float inv = 1.0f / sqrtf(ms + eps);
    for (int i = threadIdx.x; i < n; i += 256) {
        const float t = xr[i] * inv;
        o[i] = t * w[i];
    }
}

// Row r of x holds n_vec vectors of 2 * half at position pos0 + r.
__global__ __launch_bounds__(256) void rope_kernel(const float *cos_t, const float *sin_t, int half, float *x,
                                                  int n_vec, int pos0, int interleaved) {
    const int r = blockIdx.y;
    const size_t base = (size_t)(pos0 + r) * half;
    float *row = x + (size_t)r * n_vec * 2 * half;
    for (int j = blockIdx.x * 256 + threadIdx.x; j < n_vec * half; j += gridDim.x * 256) {
        const int v = j / half, i = j % half;
        float *xv = row + (size_t)v * 2 * half;
        const float c = cos_t[base + i], s = sin_t[base + i];
        const int ia = interleaved ? 2 * i : i, ib = interleaved ? 2 * i + 1 : i + half;
        const float a = xv[ia], b = xv[ib];
        const float ac = a * c, bs = b * s, bc = b * c, as = a * s;
        xv[ia] = ac - bs;
        xv[ib] = bc + as;
    }
}

__global__ __launch_bounds__(256) void swiglu_kernel(float *gate, const float *up, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float g = gate[i];
    const float silu = g / (1.0f + expf(-g));
    gate[i] = silu * up[i];
}

// One row per workgroup: max, exp(x - max), sum, times 1/sum.
__global__ __launch_bounds__(256) void softmax_kernel(float *x, int n) {
    __shared__ float s_red[256];
    float *xr = x + (size_t)blockIdx.x * n;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < n; i += 256) mx = fmaxf(mx, xr[i]);
    mx = block_max(mx, s_red);
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float e = expf(xr[i] - mx);
        xr[i] = e;
        s = s + e;
    }
    const float inv = 1.0f / block_sum(s, s_red);
    for (int i = threadIdx.x; i < n; i += 256) xr[i] = xr[i] * inv;
}

}  // namespace

int launch_swiglu(kh_ctx *ctx, float *gate, const float *up, size_t n) {
    if (n == 0) return KH_OK;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, gate, up, n);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int launch_rms_norm(kh_ctx *ctx, const float *x, const float *w, size_t m, size_t n, float eps, float *out) {
    if (m == 0 || n == 0) return KH_OK;
    hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)m), dim3(256), 0, ctx->stream, x, w, (int)n, eps, out);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

}  // namespace kh

using namespace kh;

extern "C" {

int kh_rms_norm_dev(kh_ctx *ctx, const float *x, const float *w, size_t m, size_t n, float eps, float *out) {
    if (!ctx || !x || !w || !out) return fail(KH_EINVAL, "kh_rms_norm_dev: null argument");
    if (m == 0 || n == 0) return KH_OK;
    if (m > 0x7fffffff || n > 0x7fffffff) return fail(KH_EINVAL, "kh_rms_norm_dev: too large");
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)m), dim3(256), 0, ctx->stream, x, w, (int)n, eps, out);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int kh_rope_dev(kh_ctx *ctx, const float *cos_t, const float *sin_t, size_t half, float *x, size_t m,
                size_t n_vec, size_t pos0, int interleaved) {
    if (!ctx || !cos_t || !sin_t || !x) return fail(KH_EINVAL, "kh_rope_dev: null argument");
    if (m == 0 || n_vec == 0 || half == 0) return KH_OK;
    if (m > 65535 || n_vec * half > 0x7fffffff || pos0 + m > 0x7fffffff)
        return fail(KH_EINVAL, "kh_rope_dev: too large");
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    const size_t work = n_vec * half;
    const unsigned gx = (unsigned)((work + 255) / 256 < 64 ? (work + 255) / 256 : 64);
    hipLaunchKernelGGL(rope_kernel, dim3(gx, (unsigned)m), dim3(256), 0, ctx->stream, cos_t, sin_t, (int)half, x,
                       (int)n_vec, (int)pos0, interleaved);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int kh_swiglu_dev(kh_ctx *ctx, float *gate, const float *up, size_t n) {
    if (!ctx || !gate || !up) return fail(KH_EINVAL, "kh_swiglu_dev: null argument");
    if (n == 0) return KH_OK;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    return launch_swiglu(ctx, gate, up, n);
}

int kh_softmax_dev(kh_ctx *ctx, float *x, size_t m, size_t n) {
    if (!ctx || !x) return fail(KH_EINVAL, "kh_softmax_dev: null argument");
    if (m == 0 || n == 0) return KH_OK;
    if (m > 0x7fffffff || n > 0x7fffffff) return fail(KH_EINVAL, "kh_softmax_dev: too large");
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    hipLaunchKernelGGL(softmax_kernel, dim3((unsigned)m), dim3(256), 0, ctx->stream, x, (int)n);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

}  // extern "C"
