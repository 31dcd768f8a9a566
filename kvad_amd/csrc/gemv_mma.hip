// Multi-token GEMV on the matrix cores: y[t][r] (+)= sum_b ws[r,b] xs[t,b]
// D_b[r,t] for up to 16 token rows at once (Weight::matmul_bt at a few
// tokens, crates/llm/src/quant.rs:751-907, as forward_each calls it,
// llama.rs:418-434), q8 / q4 / Q4_K weights against the rows' int8 codes.
//
// D_b, the exact i32 dot of weight row r's 32-block b with token t's codes,
// comes from the matrix core, 16 weight rows a wave:
//   - up to 8 tokens: one v_mfma_i32_16x16x64_i8 per pair of blocks.  The
//     64-wide k of the instruction spans blocks 2p and 2p+1; output columns
//     0-7 are the tokens against block 2p (their codes zero in block 2p+1's
//     k-range) and columns 8-15 the tokens against block 2p+1, so every
//     output lane holds a block dot some token needs;
//   - 9 to 16 tokens: one v_mfma_i32_16x16x32_i8 per block, a column per
//     token.
// The block's scaling follows in registers (convert, scale product, fused
// multiply-add per output).  Q4_K's minimum terms sum_j dmin m_j[r] xs[t,j]
// sum_j[t] are a true product over the sub-block index and go through
// v_mfma_f32_16x16x4_f32, four sub-blocks an instruction.
//
// Work.  A workgroup owns 16 weight rows of one job; its NW waves split the
// row's k-range into contiguous unit ranges (a unit: four 32-blocks of q8 /
// q4, one 256-wide Q4_K super-block).  Lanes load the weights and codes they
// feed the matrix core straight from memory (the codes are a few hundred KB
// at most and stay in the caches); a wave issues the loads of R units before
// it computes any, and every load is unconditional (a lane with nothing to
// read addresses past its buffer's end, which reads zeros), so each wait
// covers only the loads it needs.  Scales and block parameters, loaded one
// per lane, reach the accumulator layout (rows 4 (lane >> 4) .. + 4 of the
// lane's column) through a wave-private LDS exchange.  The waves' partial
// tiles are summed in wave order in LDS, so results do not depend on timing;
// bias and the residual add are applied once.
//
// Sums run in another order than the single-token GEMV's, so a token's row
// agrees with its matvec to rounding (1e-5 relative), not to the bit.
#include "gemv_core.hpp"

namespace kh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr unsigned XOOB = 0x80000000u;  // a base past every codes / scales buffer (< 2 GiB)
constexpr int MMA_TOKENS = 16, PAIR_TOKENS = 8;

struct MmaJob {
    const void *w;
    const float *ws;     // q8 / q4 block scales [rows][nb]; unused for Q4_K
    const float *bias;   // [rows] or null
    float *y;            // [m][rows]
    int rows, accumulate;
    int g0;              // the job's first workgroup (16 rows each)
};

struct MmaArgs {
    const int8_t *xq;     // [m][cols] codes
    const float *xs;      // [m][nb] block scales
    const int32_t *xsum;  // [m][nb] block code sums (Q4_K's minimum term)
    int cols, m, njobs;
    int units;            // per row: four-block quads (q8, q4) or super-blocks (Q4_K)
    MmaJob j[MULTI_JOBS];
};

// Orders this wave's LDS writes before its next reads (LDS serves a wave's
// requests in order; the clobber keeps the compiler from moving them).
__device__ __forceinline__ void wave_lds_sync() { __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ unsigned long long bld8(const rsrc_t &r, unsigned off) {
    return __builtin_bit_cast(unsigned long long, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}

// Four nibble codes per byte lane -> signed (code - 8) bytes, no borrows.
__device__ __forceinline__ unsigned nib_minus8(unsigned x) {
    return ((x | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

__device__ __forceinline__ v4i mma32(unsigned long long a, unsigned long long b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)a, (long)b, z, 0, 0, 0);
}
__device__ __forceinline__ v4i mma64(const int4 &a, const int4 &b) {
    const v4i z = {0, 0, 0, 0};
    const v4i va = {a.x, a.y, a.z, a.w}, vb = {b.x, b.y, b.z, b.w};
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(va, vb, z, 0, 0, 0);
}

// acc[i] += D[i] * (w[i] * x)
__device__ __forceinline__ void scale_add(v4f &acc, const v4i &D, const float4 &w, float x) {
    acc[0] = fmaf((float)D[0], w.x * x, acc[0]);
    acc[1] = fmaf((float)D[1], w.y * x, acc[1]);
    acc[2] = fmaf((float)D[2], w.z * x, acc[2]);
    acc[3] = fmaf((float)D[3], w.w * x, acc[3]);
}

// A lane's fixed addressing: lr = lane & 15, lg = lane >> 4.  Rows past the
// job's end and tokens past m address past their buffers' ends.
struct Lane {
    int lr, lg;
    unsigned wrow;   // weight row lr's first byte
    unsigned wsrow;  // its block scales (q8 / q4), bytes
    unsigned xrow;   // 16-token mode: token lr's codes; paired mode: the codes this lane feeds
    unsigned xsrow;  // token scales / sums of the lane's token, bytes
    unsigned xsrow2; // paired q8 / q4: token lr & 7's scales, bytes
};

// ---- one unit's registers, per lane --------------------------------------
template <int PREC, bool PAIR>
struct Unit;
template <>
struct Unit<KH_Q8, false> {
    unsigned long long a[4], b[4];
    float ws, xs;
};
template <>
struct Unit<KH_Q4, false> {
    unsigned a[4];
    unsigned long long b[4];
    float ws, xs;
};
template <>
struct Unit<KH_Q8, true> {  // the quad's two block pairs
    int4 a[2], b[2];
    float ws, xs;
};
template <>
struct Unit<KH_Q4, true> {
    int4 a[2], b[2];
    float ws, xs;
};
template <bool PAIR>
struct Unit<KH_Q4K, PAIR> {
    int4 h;
    typename std::conditional<PAIR, int4, unsigned long long>::type a[4];
    typename std::conditional<PAIR, int4, unsigned long long>::type b[PAIR ? 4 : 8];
    float xs[2];
    int sum[2];
};

template <int PREC, bool PAIR>
__device__ __forceinline__ void load_unit(Unit<PREC, PAIR> &u, int q, unsigned um, const Lane &L, const rsrc_t &W,
                                          const rsrc_t &WS, const rsrc_t &X, const rsrc_t &XS, const rsrc_t &XM,
                                          int nb) {
    // um: 0, or all ones for a unit past the wave's share (every load reads zeros)
    if constexpr (PREC == KH_Q4K) {
        const unsigned base = L.wrow + (unsigned)q * Q4K_BYTES;
        u.h = bld16(W, base | um);
        if constexpr (PAIR) {
            // pair c: qs bytes 32c + 16 (lg & 1) .. + 16 (sub-block 2c low, 2c+1 high nibbles)
#pragma unroll
            for (int c = 0; c < 4; c++) u.a[c] = bld16(W, (base + 16 + 32 * c + 16 * (L.lg & 1)) | um);
#pragma unroll
            for (int c = 0; c < 4; c++) u.b[c] = bld16(X, (L.xrow + (unsigned)q * QK_K + 64 * c) | um);
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++) u.a[c] = bld8(W, (base + 16 + 32 * c + 8 * L.lg) | um);
#pragma unroll
            for (int j = 0; j < 8; j++) u.b[j] = bld8(X, (L.xrow + (unsigned)q * QK_K + 32 * j + 8 * L.lg) | um);
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const unsigned o = (L.xsrow + (8 * q + 4 * h + L.lg) * 4) | um;
            u.xs[h] = bldf(XS, o);
            u.sum[h] = bldi(XM, o);
        }
    } else {
        const int b0 = 4 * q;
        if constexpr (PAIR) {
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const unsigned pb = (unsigned)(2 * q + p);
                u.a[p] = bld16(W, (PREC == KH_Q8 ? L.wrow + 64 * pb + 16 * L.lg
                                                 : L.wrow + 32 * pb + 16 * (L.lg >> 1)) | um);
                u.b[p] = bld16(X, (L.xrow + 64 * pb) | um);
            }
            u.xs = bldf(XS, (L.xsrow2 + (b0 + L.lg) * 4) | um);
        } else {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                if constexpr (PREC == KH_Q8) {
                    u.a[k] = bld8(W, (L.wrow + 32 * (b0 + k) + 8 * L.lg) | um);
                    u.b[k] = bld8(X, (L.xrow + 32 * (b0 + k) + 8 * L.lg) | um);
                } else {
                    u.a[k] = (unsigned)bldi(W, (L.wrow + 16 * (b0 + k) + 4 * L.lg) | um);
                    const unsigned tb = L.xrow + 32 * (b0 + k) + 4 * L.lg;
                    const unsigned lo = (unsigned)bldi(X, tb | um), hi = (unsigned)bldi(X, (tb + 16) | um);
                    u.b[k] = (unsigned long long)lo | ((unsigned long long)hi << 32);
                }
            }
            u.xs = bldf(XS, (L.xsrow + (b0 + L.lg) * 4) | um);
        }
        // past the row's last block the loads read the next row's bytes: the
        // scale is zeroed there, so those products add nothing
        const float w = bldf(WS, (L.wsrow + (b0 + L.lg) * 4) | um);
        u.ws = b0 + L.lg < nb ? w : 0.0f;
    }
}

// ex: this wave's 256-float exchange area.  acc: the lane's column, rows
// 4 lg .. + 4; accm: Q4_K's minimum terms (token lr's column).
template <int PREC, bool PAIR>
__device__ __forceinline__ void compute_unit(const Unit<PREC, PAIR> &u, v4f &acc, v4f &accm, float *ex,
                                             const Lane &L) {
    const int lr = L.lr, lg = L.lg;
    if constexpr (PREC == KH_Q4K) {
        // sub-blocks lg and lg + 4 of row lr: d * sc and dmin * m (mpp.rs:276-282, 304-315)
        const float d = half_bits_to_float((unsigned)u.h.x), dmin = half_bits_to_float((unsigned)u.h.x >> 16);
        float dl[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            unsigned sc, mn;
            q4k_scale_min_bfe(u.h, q4k_lane(lg + 4 * h), sc, mn);
            dl[h] = d * (float)sc;
            const float ml = dmin * (float)mn;
            // minimum terms of sub-blocks 4h .. 4h + 3: A[row][k] = ml of
            // sub-block 4h + k, B[k][tok] = xs * sum of the token's sub-block
            const float s = u.xs[h] * (float)u.sum[h];
            accm = __builtin_amdgcn_mfma_f32_16x16x4f32(ml, s, accm, 0, 0, 0);
        }
        ex[lg * 16 + lr] = dl[0];
        ex[(lg + 4) * 16 + lr] = dl[1];
        if constexpr (PAIR) {
            // [token][parity][pair]: sub-block j = 2c + p at 4p + c
            if (lr < PAIR_TOKENS) {
                ex[128 + lr * 8 + 4 * (lg & 1) + (lg >> 1)] = u.xs[0];
                ex[128 + lr * 8 + 4 * (lg & 1) + 2 + (lg >> 1)] = u.xs[1];
            }
            wave_lds_sync();
            const int t = lr & 7, p = lr >> 3;
            const float4 x4 = *reinterpret_cast<const float4 *>(ex + 128 + t * 8 + 4 * p);
            const float xk[4] = {x4.x, x4.y, x4.z, x4.w};
            const int sh = 4 * (lg >> 1);  // lanes lg < 2 feed the low nibbles (sub-block 2c), others the high
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int4 q4 = u.a[c];
                const int4 w = {(int)(((unsigned)q4.x >> sh) & 0x0f0f0f0fu), (int)(((unsigned)q4.y >> sh) & 0x0f0f0f0fu),
                                (int)(((unsigned)q4.z >> sh) & 0x0f0f0f0fu), (int)(((unsigned)q4.w >> sh) & 0x0f0f0f0fu)};
                const v4i D = mma64(w, u.b[c]);
                const float4 dl4 = *reinterpret_cast<const float4 *>(ex + (2 * c + p) * 16 + 4 * lg);
                scale_add(acc, D, dl4, xk[c]);
            }
        } else {
            ex[128 + lr * 8 + lg] = u.xs[0];
            ex[128 + lr * 8 + lg + 4] = u.xs[1];
            wave_lds_sync();
            const float4 x0 = *reinterpret_cast<const float4 *>(ex + 128 + lr * 8);
            const float4 x1 = *reinterpret_cast<const float4 *>(ex + 128 + lr * 8 + 4);
            const float xs8[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const unsigned long long q = u.a[j >> 1];
                const unsigned lo = (unsigned)q, hi = (unsigned)(q >> 32);
                const unsigned w0 = (j & 1) ? (lo >> 4) & 0x0f0f0f0fu : lo & 0x0f0f0f0fu;
                const unsigned w1 = (j & 1) ? (hi >> 4) & 0x0f0f0f0fu : hi & 0x0f0f0f0fu;
                const v4i D = mma32((unsigned long long)w0 | ((unsigned long long)w1 << 32), u.b[j]);
                const float4 dl4 = *reinterpret_cast<const float4 *>(ex + j * 16 + 4 * lg);
                scale_add(acc, D, dl4, xs8[j]);
            }
        }
        wave_lds_sync();
    } else {
        ex[lg * 16 + lr] = u.ws;  // [block][row]
        if constexpr (PAIR) {
            // [token][parity][pair]: block 2 pp + p of the quad at 2p + pp
            ex[64 + (lr & 7) * 4 + 2 * (lg & 1) + (lg >> 1)] = u.xs;
            wave_lds_sync();
            const int t = lr & 7, p = lr >> 3;
            const float2 x2 = *reinterpret_cast<const float2 *>(ex + 64 + t * 4 + 2 * p);
            const float xk[2] = {x2.x, x2.y};
#pragma unroll
            for (int pp = 0; pp < 2; pp++) {
                int4 A = u.a[pp];
                if constexpr (PREC == KH_Q4) {
                    // block 2 pb + (lg >> 1), weights 16 (lg & 1) .. + 16: low nibbles of its
                    // 16 bytes for the first half, high for the second (quant.rs:258-274)
                    const int sh = 4 * (lg & 1);
                    A = {(int)nib_minus8(((unsigned)A.x >> sh) & 0x0f0f0f0fu),
                         (int)nib_minus8(((unsigned)A.y >> sh) & 0x0f0f0f0fu),
                         (int)nib_minus8(((unsigned)A.z >> sh) & 0x0f0f0f0fu),
                         (int)nib_minus8(((unsigned)A.w >> sh) & 0x0f0f0f0fu)};
                }
                const v4i D = mma64(A, u.b[pp]);
                const float4 w4 = *reinterpret_cast<const float4 *>(ex + (2 * pp + p) * 16 + 4 * lg);
                scale_add(acc, D, w4, xk[pp]);
            }
        } else {
            ex[64 + lr * 4 + lg] = u.xs;  // [token][block]
            wave_lds_sync();
            const float4 x4 = *reinterpret_cast<const float4 *>(ex + 64 + lr * 4);
            const float xk[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                unsigned long long A;
                if constexpr (PREC == KH_Q8) {
                    A = u.a[k];
                } else {
                    // byte i: weight i (low nibble), 16 + i (high)
                    const unsigned lo = nib_minus8(u.a[k] & 0x0f0f0f0fu),
                                   hi = nib_minus8((u.a[k] >> 4) & 0x0f0f0f0fu);
                    A = (unsigned long long)lo | ((unsigned long long)hi << 32);
                }
                const v4i D = mma32(A, u.b[k]);
                const float4 w4 = *reinterpret_cast<const float4 *>(ex + k * 16 + 4 * lg);
                scale_add(acc, D, w4, xk[k]);
            }
        }
        wave_lds_sync();
    }
}

template <int PREC, bool PAIR, int NW, int R>
__global__ __launch_bounds__(WAVE * NW) void gemv_mma_kernel(unsigned g12, MmaArgs a) {
    static_assert(MULTI_JOBS == 3, "g12 holds jobs 1 and 2");
    __shared__ __align__(16) float s_ex[NW][256];
    __shared__ __align__(16) float s_red[NW][WAVE * 4];
    const int tid = threadIdx.x, lane = tid & (WAVE - 1);
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ji = ((int)blockIdx.x >= (int)(g12 & 0xffffu) ? 1 : 0) + ((int)blockIdx.x >= (int)(g12 >> 16) ? 1 : 0);
    const MmaJob &job = a.j[ji];
    // the fields the first loads need, in one batch of scalar loads
    __asm__ volatile("" ::"s"(job.w), "s"(job.ws), "s"(job.rows), "s"(job.g0), "s"(a.cols), "s"(a.m), "s"(a.units),
                     "s"(a.xq), "s"(a.xs), "s"(a.xsum));
    const int rg = (int)blockIdx.x - job.g0, rows = job.rows, nb = a.cols / BLOCK;

    Lane L;
    L.lr = lane & 15;
    L.lg = lane >> 4;
    const unsigned row_bytes = PREC == KH_Q8 ? (unsigned)a.cols
                               : PREC == KH_Q4 ? (unsigned)a.cols / 2
                                               : (unsigned)(a.cols / QK_K) * Q4K_BYTES;
    const unsigned row = (unsigned)(rg * 16 + L.lr);
    L.wrow = row * row_bytes;
    L.wsrow = row * (unsigned)nb * 4;
    if constexpr (PAIR) {
        // column lr: token lr & 7 against the pair's block lr >> 3; lane
        // group lg feeds k 16 lg .. + 16, i.e. block lg >> 1 of the pair
        L.xrow = (L.lg >> 1) == (L.lr >> 3) ? (unsigned)(L.lr & 7) * (unsigned)a.cols + 16 * L.lg : XOOB;
        L.xsrow2 = (unsigned)(L.lr & 7) * (unsigned)nb * 4;
    } else {
        L.xrow = (unsigned)L.lr * (unsigned)a.cols;
        L.xsrow2 = 0;
    }
    L.xsrow = (unsigned)L.lr * (unsigned)nb * 4;
    const rsrc_t W = rsrc(job.w, (size_t)rows * row_bytes);
    const rsrc_t WS = rsrc(job.ws, PREC == KH_Q4K ? 0 : (size_t)rows * nb * 4);
    const rsrc_t X = rsrc(a.xq, (size_t)a.m * a.cols);
    const rsrc_t XS = rsrc(a.xs, (size_t)a.m * nb * 4), XM = rsrc(a.xsum, (size_t)a.m * nb * 4);

    // this wave's units: a contiguous share of the row's k-range
    const int u0 = (int)((long long)a.units * wv / NW), u1 = (int)((long long)a.units * (wv + 1) / NW);
    v4f acc = {0.f, 0.f, 0.f, 0.f}, accm = {0.f, 0.f, 0.f, 0.f};
    float *ex = s_ex[wv];
    for (int q0 = u0; q0 < u1; q0 += R) {
        Unit<PREC, PAIR> u[R];
#pragma unroll
        for (int i = 0; i < R; i++) load_unit<PREC, PAIR>(u[i], q0 + i, q0 + i < u1 ? 0u : ~0u, L, W, WS, X, XS, XM, nb);
#pragma unroll
        for (int i = 0; i < R; i++)
            if (q0 + i < u1) compute_unit<PREC, PAIR>(u[i], acc, accm, ex, L);
    }
    if constexpr (PREC == KH_Q4K) acc -= accm;  // paired: accm is zero in columns 8-15
    *reinterpret_cast<v4f *>(&s_red[wv][lane * 4]) = acc;
    __syncthreads();
    if (wv != 0) return;
    v4f s = *reinterpret_cast<const v4f *>(&s_red[0][lane * 4]);
    for (int w = 1; w < NW; w++) s += *reinterpret_cast<const v4f *>(&s_red[w][lane * 4]);
    if constexpr (PAIR) {
        // column lr + 8 holds the same token against the pairs' odd blocks.
        // Added through LDS: a DPP row rotate of the vector's elements was
        // miscompiled (only element 0 rotated, the others read its result).
        if (L.lr < PAIR_TOKENS)
            for (int w = 0; w < NW; w++) s += *reinterpret_cast<const v4f *>(&s_red[w][(lane + 8) * 4]);
    }
    const int tok = L.lr;
    if (tok >= a.m || (PAIR && tok >= PAIR_TOKENS)) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = rg * 16 + 4 * L.lg + i;
        if (r < rows) {
            float *dst = job.y + (size_t)tok * rows + r;
            const float o = job.bias ? s[i] + job.bias[r] : s[i];
            *dst = job.accumulate ? *dst + o : o;  // x += proj (llama.rs:273-276)
        }
    }
}

template <int PREC, bool PAIR, int R>
int launch_nw(kh_ctx *ctx, const MmaArgs &a, int nwg, int nw) {
    if (nwg >= 0xffff) return fail(KH_DECLINED, "matmul: 65535 workgroups or more in one launch");
    const unsigned g12 = multi_firsts(a.njobs, a.j[1].g0, a.j[2].g0);
    if (nw == 16)
        hipLaunchKernelGGL((gemv_mma_kernel<PREC, PAIR, 16, R>), dim3(nwg), dim3(WAVE * 16), 0, ctx->stream, g12, a);
    else if (nw == 8)
        hipLaunchKernelGGL((gemv_mma_kernel<PREC, PAIR, 8, R>), dim3(nwg), dim3(WAVE * 8), 0, ctx->stream, g12, a);
    else
        hipLaunchKernelGGL((gemv_mma_kernel<PREC, PAIR, 4, R>), dim3(nwg), dim3(WAVE * 4), 0, ctx->stream, g12, a);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

template <int PREC, int R>
int launch_mode(kh_ctx *ctx, const MmaArgs &a, int nwg, int nw) {
    return a.m <= PAIR_TOKENS ? launch_nw<PREC, true, R>(ctx, a, nwg, nw) : launch_nw<PREC, false, R>(ctx, a, nwg, nw);
}

}  // namespace

int launch_gemv_mma(kh_ctx *ctx, int njobs, const kh_weight *const *w, const float *const *bias, float *const *y,
                    const int *accumulate, const QAct &x, size_t m) {
    if (m == 0) return KH_OK;
    if (njobs < 1 || njobs > MULTI_JOBS) return fail(KH_EINVAL, "matmul: one to three weights per launch");
    const int prec = w[0]->precision;
    const size_t cols = w[0]->cols;
    if (prec != KH_Q8 && prec != KH_Q4 && prec != KH_Q4K)
        return fail(KH_EINVAL, "matmul: the matrix-core GEMV takes quantised weights");
    if (cols % (prec == KH_Q4K ? QK_K : BLOCK)) return fail(KH_EINVAL, "matmul: width not a whole number of blocks");
    if (MMA_TOKENS * cols >= XOOB) return fail(KH_DECLINED, "matmul: rows of codes of 128 MB or more");
    MmaArgs a{};
    a.cols = (int)cols;
    a.njobs = njobs;
    const int nb = (int)(cols / BLOCK);
    a.units = prec == KH_Q4K ? (int)(cols / QK_K) : (nb + 3) / 4;
    int nwg = 0;
    for (int i = 0; i < njobs; i++) {
        if (w[i]->precision != prec || w[i]->cols != cols)
            return fail(KH_EINVAL, "matmul: weights of one launch share precision and width");
        const size_t rb = prec == KH_Q8 ? cols : prec == KH_Q4 ? cols / 2 : cols / QK_K * Q4K_BYTES;
        // rows past the end (up to 15) still address below 4 GiB
        if ((w[i]->rows + 16) * rb >= 0xfff00000ull || (w[i]->rows + 16) * (cols / BLOCK) * 4 >= 0xfff00000ull)
            return fail(KH_DECLINED, "matmul: operands of 4 GiB or more are not addressed here");
        a.j[i] = MmaJob{w[i]->qs, w[i]->scales, bias ? bias[i] : nullptr, y[i], (int)w[i]->rows,
                        accumulate ? accumulate[i] : 0, nwg};
        nwg += (int)((w[i]->rows + 15) / 16);
    }
    // Four waves per workgroup, each taking several rounds of R units when
    // the rows are long: measured at or ahead of 8 and 16 waves at every
    // shape (m = 8, us for 4 / 8 / 16 waves: Q4_K 14336x4096 23.1 / 22.8 /
    // 33.3, 4096x14336 20.7 / 21.2 / 21.9; q8 896x4864 10.8 / 11.3 / 11.9,
    // 151936x896 49.4 / 78.1 / 91.9)
    int nw = 4;
    const int forced = env_int("KVAD_MMA_WAVES", 0);  // tuning knob
    if (forced == 4 || forced == 8 || forced == 16) nw = forced;
    for (size_t t0 = 0; t0 < m; t0 += MMA_TOKENS) {
        MmaArgs b = a;
        b.m = (int)(m - t0 < (size_t)MMA_TOKENS ? m - t0 : MMA_TOKENS);
        b.xq = x.qs + t0 * cols;
        b.xs = x.scales + t0 * nb;
        b.xsum = x.sums + t0 * nb;
        for (int i = 0; i < njobs; i++) b.j[i].y = a.j[i].y + t0 * a.j[i].rows;
        int rc;
        // two units a round (measured against 1, 4 and 8 at m = 8: q8
        // 151936x896 37.2 against 49.5 us at 4; Q4_K level with 1, 4 slower)
        switch (prec) {
            case KH_Q8: rc = launch_mode<KH_Q8, 2>(ctx, b, nwg, nw); break;
            case KH_Q4: rc = launch_mode<KH_Q4, 2>(ctx, b, nwg, nw); break;
            default: rc = launch_mode<KH_Q4K, 2>(ctx, b, nwg, nw); break;
        }
        if (rc) return rc;
    }
    return KH_OK;
}

}  // namespace kh
