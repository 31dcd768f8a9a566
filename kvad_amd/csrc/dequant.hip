// The dequantising single-token GEMV: Weight::matvec_bt_dequant
// (crates/llm/src/quant.rs:522-589), which the reference keeps as the
// baseline of its integer path and selects with KVAD_DEQUANT=1
// (quant.rs:592-610).  Weights are unpacked to f32 in registers and
// multiplied with the f32 activation as it is: no quantisation of x, no LDS
// stage, no workgroup barrier before the first weight is used.
//
// Shape of the kernel.  A wave owns R rows at a time and walks them together
// in 16-byte weight chunks, lane l taking chunks l, l + 64, ... (q8: half a
// 32-block; q4: one block; Q4_K: half of two sub-blocks' nibbles), so one load
// instruction moves 1 KiB of contiguous weight bytes.  The activation values
// a chunk meets are read straight from global memory (the L1/L2 keep the
// vector, a few KiB to 57 KiB, resident for every wave) and shared by the R
// rows.  Loads are buffer loads: reads past the end of the activation return
// zeros, so a chunk past the end of a row contributes nothing and tails need
// no branch.
//
// Arithmetic.  q8: the reference's per-block sum of x * (f32)q, scaled by the
// block scale.  q4: sum of x * nibble minus 8 * sum(x) per block
// (quant.rs:571-577); the high nibbles are taken in place (16 * code, an
// exact power-of-two scaling undone by one multiply).  Q4_K: per 32-wide
// sub-block d * sc * sum(x * q) - dmin * m * sum(x), the form of
// gpu/src/mpp.rs:304-315 with the sums over x.  Products are fused
// multiply-adds and sums run in lane order, so outputs match the reference to
// f32 rounding (1e-5 relative to the largest output), not to the bit.
#include <cstring>

#include "common.hpp"
#include "device.hpp"

namespace kh {
namespace {

using namespace dev;

constexpr int DQ_WAVES = 4;  // waves per workgroup

struct DqArgs {
    const void *w;       // q8 int8 / q4 packed / Q4_K blocks
    const float *ws;     // q8/q4 block scales (null for Q4_K)
    const float *x;      // f32 activation [cols]
    const float *bias;   // [rows] or null
    float *y;            // [rows]
    int rows, cols, nwaves;
};

__host__ __device__ inline int dq_chunks(int prec, int cols) {
    return prec == KH_Q8 ? cols / 16 : prec == KH_Q4 ? cols / 32 : (cols / QK_K) * 8;
}

// Byte k of w as a signed integer, as f32.
__device__ __forceinline__ float sbyte(int w, int k) { return (float)((w << (24 - 8 * k)) >> 24); }

// sum_k code_k * x_k over the four bytes of `c` (unsigned codes) and a
// float4; each byte converts with one v_cvt_f32_ubyteN.
__device__ __forceinline__ float udot4f(unsigned c, float4 x, float f) {
    f = fmaf((float)(c & 0xffu), x.x, f);
    f = fmaf((float)((c >> 8) & 0xffu), x.y, f);
    f = fmaf((float)((c >> 16) & 0xffu), x.z, f);
    f = fmaf((float)(c >> 24), x.w, f);
    return f;
}
__device__ __forceinline__ float sdot4f(int c, float4 x, float f) {
    f = fmaf(sbyte(c, 0), x.x, f);
    f = fmaf(sbyte(c, 1), x.y, f);
    f = fmaf(sbyte(c, 2), x.z, f);
    f = fmaf(sbyte(c, 3), x.w, f);
    return f;
}
__device__ __forceinline__ float hsum4(float4 v) { return (v.x + v.y) + (v.z + v.w); }

// One step's loads: R rows' chunk of the weights and the activation values
// it meets.
template <int PREC, int R>
struct DqStep {
    int4 w[R];
    int4 hd[PREC == KH_Q4K ? R : 1];   // Q4_K block headers
    float s[PREC == KH_Q4K ? 1 : R];   // q8/q4 block scales
    float4 xl[4];
    float4 xh[PREC == KH_Q8 ? 1 : 4];
};

template <int PREC, int R>
__device__ __forceinline__ void dq_load(DqStep<PREC, R> &st, const rsrc_t &W, const rsrc_t &WS, const rsrc_t &X,
                                        int r0, unsigned g, int cols, int nb, int lane, int cq, int h) {
    if constexpr (PREC == KH_Q8) {
        // weights 16g .. 16g + 15, block g / 2
#pragma unroll
        for (int k = 0; k < 4; k++) st.xl[k] = bld16f(X, g * 64 + 16 * k);
#pragma unroll
        for (int i = 0; i < R; i++) {
            const unsigned r = (unsigned)(r0 + i);
            st.w[i] = bld16(W, r * (unsigned)cols + g * 16);
            st.s[i] = bldf(WS, (r * (unsigned)nb + (g >> 1)) * 4);
        }
    } else if constexpr (PREC == KH_Q4) {
        // block g: byte k holds weight k (low nibble) and k + 16 (high)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            st.xl[k] = bld16f(X, g * 128 + 16 * k);
            st.xh[k] = bld16f(X, g * 128 + 64 + 16 * k);
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            const unsigned r = (unsigned)(r0 + i);
            st.w[i] = bld16(W, r * (unsigned)(cols / 2) + g * 16);
            st.s[i] = bldf(WS, (r * (unsigned)nb + g) * 4);
        }
    } else {
        // Q4_K chunk g: block g / 8, qs bytes 32c + 16h .. + 15
        const unsigned xb = (g >> 3) * QK_K + 64 * cq + 16 * h;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            st.xl[k] = bld16f(X, (xb + 4 * k) * 4);
            st.xh[k] = bld16f(X, (xb + 32 + 4 * k) * 4);
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            const unsigned r = (unsigned)(r0 + i);
            const unsigned bo = r * (unsigned)((cols / QK_K) * Q4K_BYTES) + (g >> 3) * Q4K_BYTES;
            st.hd[i] = bld16(W, bo);
            st.w[i] = bld16(W, bo + 16 + 16 * (unsigned)(lane & 7));
        }
    }
}

template <int PREC, int R>
__device__ __forceinline__ void dq_compute(const DqStep<PREC, R> &st, float (&acc)[R], int h, int sh,
                                           unsigned hij) {
    if constexpr (PREC == KH_Q8) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            float f = sdot4f(st.w[i].x, st.xl[0], 0.0f);
            f = sdot4f(st.w[i].y, st.xl[1], f);
            f = sdot4f(st.w[i].z, st.xl[2], f);
            f = sdot4f(st.w[i].w, st.xl[3], f);
            acc[i] = fmaf(st.s[i], f, acc[i]);
        }
    } else if constexpr (PREC == KH_Q4) {
        const float xsum = ((hsum4(st.xl[0]) + hsum4(st.xl[1])) + (hsum4(st.xl[2]) + hsum4(st.xl[3]))) +
                           ((hsum4(st.xh[0]) + hsum4(st.xh[1])) + (hsum4(st.xh[2]) + hsum4(st.xh[3])));
#pragma unroll
        for (int i = 0; i < R; i++) {
            const unsigned q[4] = {(unsigned)st.w[i].x, (unsigned)st.w[i].y, (unsigned)st.w[i].z,
                                   (unsigned)st.w[i].w};
            float lo = 0.0f, hi = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                lo = udot4f(q[k] & 0x0f0f0f0fu, st.xl[k], lo);
                hi = udot4f(q[k] & 0xf0f0f0f0u, st.xh[k], hi);  // 16 * code
            }
            const float dot = fmaf(hi, 0.0625f, lo) - 8.0f * xsum;
            acc[i] = fmaf(st.s[i], dot, acc[i]);
        }
    } else {
        // sum of x over the lane's sub-block: its 16 values and its partner's
        float sl = (hsum4(st.xl[0]) + hsum4(st.xl[1])) + (hsum4(st.xl[2]) + hsum4(st.xl[3]));
        float su = (hsum4(st.xh[0]) + hsum4(st.xh[1])) + (hsum4(st.xh[2]) + hsum4(st.xh[3]));
        sl = sl + dppf<DPP_XOR1>(sl);  // a + b == b + a: both lanes agree
        su = su + dppf<DPP_XOR1>(su);
        const float xs = h ? su : sl;
#pragma unroll
        for (int i = 0; i < R; i++) {
            const unsigned q[4] = {(unsigned)st.w[i].x, (unsigned)st.w[i].y, (unsigned)st.w[i].z,
                                   (unsigned)st.w[i].w};
            float lo = 0.0f, hi = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                lo = udot4f(q[k] & 0x0f0f0f0fu, st.xl[k], lo);
                hi = udot4f(q[k] & 0xf0f0f0f0u, st.xh[k], hi);  // 16 * code
            }
            lo = lo + dppf<DPP_XOR1>(lo);
            hi = hi + dppf<DPP_XOR1>(hi);
            const float f = h ? hi * 0.0625f : lo;
            unsigned sc, mn;
            q4k_scale_min(st.hd[i], sh, hij, sc, mn);
            const float dl = half_bits_to_float((unsigned)st.hd[i].x) * (float)sc;
            const float ml = half_bits_to_float((unsigned)st.hd[i].x >> 16) * (float)mn;
            acc[i] = acc[i] + (dl * f - ml * xs);
        }
    }
}

// The wave's work is a sequence of steps: row group lw + (s / nt) * nw, chunk
// column s % nt.  Two register sets take even and odd steps, and every pass
// of the loop issues the same loads (a step past the wave's work reads past
// the end of the weights, which returns zeros), so a step waits only for its
// own loads while the next step's are in flight.
template <int PREC, int R>
__global__ __launch_bounds__(WAVE * DQ_WAVES) void gemv_dq_kernel(DqArgs a) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int lw = blockIdx.x * DQ_WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rows = a.rows, cols = a.cols, nb = cols / BLOCK, nw = a.nwaves;
    const int C = dq_chunks(PREC, cols);
    const int nt = (C + WAVE - 1) / WAVE;  // chunk columns per lane per row
    const size_t wbytes = PREC == KH_Q8 ? (size_t)rows * cols
                          : PREC == KH_Q4 ? (size_t)rows * cols / 2
                                          : (size_t)rows * (cols / QK_K) * Q4K_BYTES;
    const rsrc_t W = rsrc(a.w, wbytes);
    const rsrc_t WS = rsrc(a.ws, PREC == KH_Q4K ? 0 : (size_t)rows * nb * 4);
    const rsrc_t X = rsrc(a.x, (size_t)cols * 4);
    // Q4_K: the sub-blocks a lane's chunk holds are fixed by the lane
    // (64 % 8 == 0): low nibbles of 2c, high nibbles of 2c + 1, positions
    // 16h..16h+15 of each; the lane finishes sub-block j = 2c + h.
    const int h = lane & 1, cq = (lane & 7) >> 1, j = 2 * cq + h;
    const int sh = 8 * (j & 3);
    const unsigned hij = j >= 4 ? ~0u : 0u;

    const int ngroups = (rows + R - 1) / R;
    const int my_groups = lw < ngroups ? (ngroups - lw + nw - 1) / nw : 0;
    const int steps = my_groups * nt;
    auto load_step = [&](DqStep<PREC, R> &st, int s) {
        __builtin_amdgcn_sched_barrier(0);
        dq_load<PREC, R>(st, W, WS, X, (lw + (s / nt) * nw) * R, (unsigned)((s % nt) * WAVE + lane), cols, nb,
                         lane, cq, h);
        __builtin_amdgcn_sched_barrier(0);
    };
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++) acc[i] = 0.0f;
    auto run_step = [&](const DqStep<PREC, R> &st, int s) {
        dq_compute<PREC, R>(st, acc, h, sh, hij);
        if (s % nt == nt - 1) {
            const int r0 = (lw + (s / nt) * nw) * R;
#pragma unroll
            for (int i = 0; i < R; i++) {
                const float v = wave_sum(acc[i]);
                const int r = r0 + i;
                if (lane == 0 && r < rows) a.y[r] = a.bias ? v + a.bias[r] : v;
                acc[i] = 0.0f;
            }
        }
    };
    DqStep<PREC, R> ca, cb;
    load_step(ca, 0);
    for (int s = 0; s < steps; s += 2) {
        load_step(cb, s + 1);
        run_step(ca, s);
        load_step(ca, s + 2);
        if (s + 1 < steps) run_step(cb, s + 1);
    }
}

template <int PREC, int R>
int launch_dq_r(kh_ctx *ctx, DqArgs a) {
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const int groups = (a.rows + R - 1) / R;
    int blocks = (groups + DQ_WAVES - 1) / DQ_WAVES;
    const int cap = env_int("KVAD_DQ_WG_PER_CU", 4) * cu;  // workgroups per CU in one round
    if (blocks > cap) blocks = cap;
    a.nwaves = blocks * DQ_WAVES;
    hipLaunchKernelGGL((gemv_dq_kernel<PREC, R>), dim3(blocks), dim3(WAVE * DQ_WAVES), 0, ctx->stream, a);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

}  // namespace

int launch_gemv_dequant(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y) {
    if (w->precision == KH_F32) return fail(KH_EINVAL, "matvec_dequant: f32 weights have nothing to dequantise");
    const size_t wb = w->precision == KH_Q8 ? w->rows * w->cols
                      : w->precision == KH_Q4 ? w->rows * w->cols / 2
                                              : w->rows * (w->cols / QK_K) * Q4K_BYTES;
    if (wb >= 0xfff00000ull || 4 * w->cols >= 0xfff00000ull)
        return fail(KH_DECLINED, "matvec_dequant: operands of 4 GiB or more are not addressed here");
    DqArgs a{w->qs, w->scales, x, bias, y, (int)w->rows, (int)w->cols, 0};
    // rows per wave step share each activation read: four for q8, two for
    // the nibble formats (whose steps hold twice the activation registers)
    switch (w->precision) {
        case KH_Q8: return launch_dq_r<KH_Q8, 4>(ctx, a);
        case KH_Q4: return launch_dq_r<KH_Q4, 2>(ctx, a);
        case KH_Q4K: return launch_dq_r<KH_Q4K, 2>(ctx, a);
        default: return fail(KH_EINVAL, "matvec_dequant: unknown precision");
    }
}

bool dequant_selected() {
    const char *e = getenv("KVAD_DEQUANT");
    return e && (!strcmp(e, "1") || !strcmp(e, "true"));
}

}  // namespace kh
