// Batched prefill GEMM on CDNA4 matrix cores: Weight::matmul_bt
// (crates/llm/src/quant.rs:751-907, x86 row_dot path) for q8 / q4 / Q4_K
// weights, and tensor::gemm_bt (tensor.rs:102-186) for f32 weights.
//
// Quantised weights.  y[m, r] = sum_b ws[r,b] * xs[m,b] * D_b[r,m] where
// D_b is the exact i32 dot of weight row r's 32-block b with token m's
// quantised block (row_dot pass 1, quant.rs:876-897).  One
// v_mfma_i32_32x32x32_i8 computes D_b for a 32x32 (rows x tokens) tile and
// exactly one 32-wide block, so every block dot is the reference's integer;
// the block's scaling (pass 2, quant.rs:899-905) is applied to the tile in
// registers before the next block.  q4 nibbles are widened to (code - 8) in
// LDS (the same integers as q4_row_dots, quant.rs:168-189); Q4_K codes are
// widened unsigned and their sub-block scale/min terms applied as the GEMV
// does (y += xs * (d*sc*dot - dmin*m*sum), mpp.rs:304-315).
//
// The per-block scaling is the bound: with 32-wide scale blocks on both
// operands every output takes a scaled term per block.  The scale products
// ws[r] * xs[t] of a tile are an outer product, computed on the matrix core,
// two tiles per v_mfma_f32_32x32x1_2b_f32 (half the matrix-core time of one
// 32x32x2 product per tile with a k-slot zeroed); Q4_K's minimum terms
// sum_b dmin*m * xs*sum are a true product over the block index and go into
// the accumulators by MFMA as well.  Two VALU operations per output per
// block remain (convert the i32 dot, fused multiply-add); matrix-core
// results are kept in VGPRs (-mllvm -amdgpu-mfma-vgpr-form), where the
// epilogue reads them without a copy.
//
// Tiles.  A workgroup of 4 waves computes a BN x BM (weight rows x tokens)
// tile; each wave WR/WT-splits it into RT x TT MFMA tiles of 32 x 32.  A
// stage is 128 k-values (4 blocks): weight and activation bytes go global ->
// registers (next stage, in flight during compute) -> LDS (rows padded by 16
// bytes), with the stage's scales beside them.  Buffer loads return zeros
// past the end of an array, so edge tiles need no branches on rows or
// tokens; a k tail (K % 128 != 0) is masked explicitly.
//
// f32 weights use v_mfma_f32_32x32x2_f32 over 32-wide k stages with the same
// tile map.  Sums are taken in a different order from the reference's
// 4-lane register tiles, so results agree to rounding (1e-5 relative).
#include <algorithm>

#include "common.hpp"

namespace kh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));


constexpr unsigned RSRC_WORD3 = 0x00020000;  // raw buffer, gfx9 family
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t rsrc(const void *p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)(bytes > 0xffffffffu ? 0xffffffffu : bytes), RSRC_WORD3);
}
__device__ __forceinline__ int4 ld16(const rsrc_t &r, unsigned off) {
    return __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float ldf(const rsrc_t &r, unsigned off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ int ldi(const rsrc_t &r, unsigned off) {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

__device__ __forceinline__ float half_bits_to_float(unsigned h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffff));
}

// Four nibble codes per byte lane -> signed (code - 8) bytes, no borrows.
__device__ __forceinline__ int nib_minus8(int x) {
    return (int)((((unsigned)x | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
}


constexpr int THREADS = 256;
constexpr int BK = 128;              // k per stage (bytes of int8)
constexpr int NBS = BK / BLOCK;      // 32-blocks per stage
constexpr int ASTR = BK + 16;        // LDS row stride, bytes

// A wave's RT x TT tiles when all of them lie inside the output (and the
// output and bias are 16-byte aligned with rows a multiple of 4 wide): one
// float4 per four rows, no per-element bounds and no branches.  dst is the
// output (bias and accumulate as store_tiles) or a split's partial plane
// (neither).  Returns false, having written nothing, otherwise.
template <int RT, int TT>
__device__ __forceinline__ bool store_tiles_full(const GemmArgs &a, float *dst, bool partial, const v16f (&acc)[RT][TT],
                                                 int r_base, int t_base, int t_end, int lane) {
    const float *bias = partial ? nullptr : a.bias;
    const bool accumulate = !partial && a.accumulate;
    if ((a.N & 3) || r_base + RT * 32 > a.N || t_base + TT * 32 > t_end ||
        (((uintptr_t)dst | (uintptr_t)bias) & 15))
        return false;
    const rsrc_t Y = rsrc(dst + (size_t)t_base * a.N + r_base, ((size_t)(TT * 32 - 1) * a.N + RT * 32) * 4);
    float4 bv[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int g = 0; g < 4; g++)
            bv[rt][g] = bias ? *reinterpret_cast<const float4 *>(bias + r_base + rt * 32 + 8 * g + 4 * (lane >> 5))
                             : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const unsigned off = ((unsigned)(tt * 32 + (lane & 31)) * (unsigned)a.N +
                                      (unsigned)(rt * 32 + 8 * g + 4 * (lane >> 5))) * 4u;
                float4 v = make_float4(acc[rt][tt][4 * g], acc[rt][tt][4 * g + 1], acc[rt][tt][4 * g + 2],
                                       acc[rt][tt][4 * g + 3]);
                if (!partial) {  // + bias (0 without one), finish, quant.rs:849-858
                    const float4 b = bv[rt][g];
                    v = make_float4(v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w);
                }
                if (accumulate) {  // x += proj (llama.rs:273-276)
                    const float4 o = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(Y, off, 0, 0));
                    v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
                }
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, v), Y, off, 0, 0);
            }
    return true;
}

// Writes a 32x32 accumulator tile (lane: token l&31, rows 8g + 4(l>>5) + e).
template <int RT, int TT>
__device__ __forceinline__ void store_tiles(const GemmArgs &a, const v16f (&acc)[RT][TT], int r_base, int t_base,
                                            int t_end, int lane) {
    if (store_tiles_full<RT, TT>(a, a.y, false, acc, r_base, t_base, t_end, lane)) return;
    const bool vec = (a.N & 3) == 0;
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            const int tok = t_base + tt * 32 + (lane & 31);
            if (tok >= t_end) continue;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int r = r_base + rt * 32 + 8 * g + 4 * (lane >> 5);
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float add = a.bias && r + e < a.N ? a.bias[r + e] : 0.0f;  // finish, quant.rs:849-858
                    v[e] = acc[rt][tt][4 * g + e] + add;
                }
                float *dst = a.y + (size_t)tok * a.N + r;
                if (vec && r + 3 < a.N) {
                    if (a.accumulate) {  // x += proj (llama.rs:273-276)
                        const float4 o = *reinterpret_cast<const float4 *>(dst);
                        v[0] = o.x + v[0], v[1] = o.y + v[1], v[2] = o.z + v[2], v[3] = o.w + v[3];
                    }
                    *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (r + e < a.N) dst[e] = a.accumulate ? dst[e] + v[e] : v[e];
                }
            }
        }
}

// Split-K: split z writes its tile's sums, unscaled by bias or residual, to
// part[z][M][N]; split_reduce_kernel, launched next, adds the splits.
template <int RT, int TT>
__device__ __forceinline__ void store_partials(const GemmArgs &a, const v16f (&acc)[RT][TT], int r_base, int t_base,
                                               int t_end, int lane) {
    const size_t plane = (size_t)a.M * a.N;
    float *part = a.part + blockIdx.z * plane;
    if (store_tiles_full<RT, TT>(a, part, true, acc, r_base, t_base, t_end, lane)) return;
    const bool vec = (a.N & 3) == 0;
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            const int tok = t_base + tt * 32 + (lane & 31);
            if (tok >= t_end) continue;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int r = r_base + rt * 32 + 8 * g + 4 * (lane >> 5);
                float *dst = part + (size_t)tok * a.N + r;
                if (vec && r + 3 < a.N) {
                    *reinterpret_cast<float4 *>(dst) = make_float4(acc[rt][tt][4 * g], acc[rt][tt][4 * g + 1],
                                                                   acc[rt][tt][4 * g + 2], acc[rt][tt][4 * g + 3]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (r + e < a.N) dst[e] = acc[rt][tt][4 * g + e];
                }
            }
        }
}

// Split-K's second launch: y = part[0] + part[1] + ... (split order), then
// bias and residual as store_tiles.  One thread per four outputs.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float *part, int ks, int M, int N,
                                                           const float *bias, int accumulate, float *y) {
    const size_t plane = (size_t)M * N, e0 = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (e0 >= plane) return;
    if ((N & 3) == 0) {  // the four outputs share a token
        const rsrc_t PT = rsrc(part, (size_t)ks * plane * 4);
        const unsigned o = (unsigned)(e0 * 4), step = (unsigned)(plane * 4);
        // every split's load in flight at once (up to 32; those past ks read
        // outside the buffer, as zeros), then the adds in split order
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int z0 = 0; z0 < ks; z0 += 32) {
            float4 p[32];
#pragma unroll
            for (int j = 0; j < 32; j++)
                p[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      PT, z0 + j < ks ? o + (z0 + j) * step : 0xffffffffu, 0, 0));
#pragma unroll
            for (int j = 0; j < 32; j++)
                if (z0 + j < ks) x = make_float4(x.x + p[j].x, x.y + p[j].y, x.z + p[j].z, x.w + p[j].w);
        }
        const int r = (int)(e0 % N);
        float v[4] = {x.x, x.y, x.z, x.w};
        if (bias) {  // finish, quant.rs:849-858
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = v[e] + bias[r + e];
        }
        float4 *dst = reinterpret_cast<float4 *>(y + e0);
        if (accumulate) {  // x += proj (llama.rs:273-276)
            const float4 o4 = *dst;
            v[0] = o4.x + v[0], v[1] = o4.y + v[1], v[2] = o4.z + v[2], v[3] = o4.w + v[3];
        }
        *dst = make_float4(v[0], v[1], v[2], v[3]);
        return;
    }
    for (int e = 0; e < 4 && e0 + e < plane; e++) {
        float x = 0.f;
        for (int z = 0; z < ks; z++) x = x + part[z * plane + e0 + e];
        const int r = (int)((e0 + e) % N);
        if (bias) x = x + bias[r];
        y[e0 + e] = accumulate ? y[e0 + e] + x : x;
    }
}

// ---------------------------------------------------------------------------
// int8 MFMA GEMM for q8 / q4 / Q4_K weights
// ---------------------------------------------------------------------------

template <int PREC, int WR, int WT, int RT, int TT>
__global__ __launch_bounds__(THREADS) void gemm_i8_kernel(GemmArgs a) {
    static_assert(WR * WT == 4, "four waves");
    constexpr int BN = WR * RT * 32, BM = WT * TT * 32;
    // per-thread global chunk counts of one stage
    constexpr int A_CH = PREC == KH_Q8 ? BN * (BK / 16) : BN * NBS;  // q4 / Q4_K: one 16-byte chunk per block
    constexpr int A_PT = (A_CH + THREADS - 1) / THREADS;
    constexpr int B_CH = BM * (BK / 16);
    constexpr int B_PT = (B_CH + THREADS - 1) / THREADS;
    constexpr int WS_PT = (BN * NBS + THREADS - 1) / THREADS;
    constexpr int XS_PT = (BM * NBS + THREADS - 1) / THREADS;

    __shared__ __align__(16) int8_t sA[BN * ASTR];
    __shared__ __align__(16) int8_t sB[BM * ASTR];
    __shared__ __align__(16) float sW[NBS][BN];   // ws (q8/q4) or d*sc (Q4_K)
    __shared__ __align__(16) float sWm[NBS][BN];  // dmin*m (Q4_K)
    __shared__ float sX[NBS][BM];                 // xs
    __shared__ float sXs[NBS][BM];                // xs * block sum (Q4_K)

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr0 = (wave / WT) * RT * 32, wm0 = (wave % WT) * TT * 32;
    const int K = a.K, nb = K / BLOCK;
    // a paired launch: row tiles past the first weight's are the second's
    const int nx = (a.N + BN - 1) / BN;
    const bool second = a.y2 && (int)blockIdx.x >= nx;
    const int n0 = ((int)blockIdx.x - (second ? nx : 0)) * BN;
    if (second) {
        a.w = a.w2, a.ws = a.ws2, a.wtab = a.wtab2, a.wstab = a.wstab2, a.y = a.y2;
        if (a.ksplit > 1) a.part += (size_t)a.ksplit * a.M * a.N;
    }

    // the workgroup's rows of activations (and, grouped, its expert)
    int m0, m_end;
    const void *wp = a.w;
    const float *wsp = a.ws;
    if (a.tiles) {
        const int t = blockIdx.y;
        if (t >= a.tiles[0]) return;  // the grid is sized for the most tiles grouping can make
        const int x = a.tiles[1 + 3 * t];
        m0 = a.tiles[2 + 3 * t];
        m_end = m0 + a.tiles[3 + 3 * t];
        wp = a.wtab[x];
        wsp = a.wstab[x];
    } else {
        m0 = blockIdx.y * BM;
        m_end = a.M;
    }

    const size_t wbytes = PREC == KH_Q8 ? (size_t)a.N * K
                          : PREC == KH_Q4 ? (size_t)a.N * K / 2
                                          : (size_t)a.N * (K / QK_K) * Q4K_BYTES;
    const rsrc_t W = rsrc(wp, wbytes);
    const rsrc_t WS = rsrc(wsp, PREC == KH_Q4K ? 0 : (size_t)a.N * nb * 4);
    const rsrc_t X = rsrc(a.xq, (size_t)a.M * K);
    const rsrc_t XS = rsrc(a.xs, (size_t)a.M * nb * 4);
    const rsrc_t XSUM = rsrc(a.xsum, PREC == KH_Q4K ? (size_t)a.M * nb * 4 : 0);

    // source activation row of each of this thread's chunks (-1: none)
    int brow[B_PT], srow[XS_PT];
#pragma unroll
    for (int u = 0; u < B_PT; u++) {
        const int r = m0 + ((tid + u * THREADS) >> 3);
        brow[u] = tid + u * THREADS < B_CH && r < m_end ? (a.gather ? a.gather[r] : r) : -1;
    }
#pragma unroll
    for (int u = 0; u < XS_PT; u++) {
        const int r = m0 + (tid + u * THREADS) / NBS;
        srow[u] = tid + u * THREADS < BM * NBS && r < m_end ? (a.gather ? a.gather[r] : r) : -1;
    }

    int4 ra[A_PT], rb[B_PT], rh;
    float rws[WS_PT], rxs[XS_PT], rxsum[XS_PT];

    // Every load is issued, the ones past a tail with an offset past the
    // buffer's end, which reads zeros: no branch around any load.
    constexpr unsigned OOB = 0xffffffffu;
    auto load_stage = [&](int k0) {
#pragma unroll
        for (int u = 0; u < A_PT; u++) {
            const int c = tid + u * THREADS;
            unsigned off;
            if constexpr (PREC == KH_Q8) {
                const int row = c >> 3, kc = c & 7;
                off = c < A_CH && k0 + 16 * kc < K ? (unsigned)(n0 + row) * (unsigned)K + (unsigned)(k0 + 16 * kc) : OOB;
            } else if constexpr (PREC == KH_Q4) {
                const int row = c / NBS, blk = c % NBS;
                off = c < A_CH && k0 / BLOCK + blk < nb
                          ? (unsigned)(n0 + row) * (unsigned)(K / 2) + (unsigned)((k0 / BLOCK + blk) * 16)
                          : OOB;
            } else {
                const int row = c / NBS, q = c % NBS;
                const unsigned sb = (unsigned)(k0 / QK_K), h = (unsigned)((k0 % QK_K) / BK);
                off = c < A_CH ? (unsigned)(n0 + row) * (unsigned)(K / QK_K) * Q4K_BYTES + sb * Q4K_BYTES + 16 +
                                     64 * h + 16 * q
                               : OOB;
            }
            ra[u] = ld16(W, off);
        }
        if constexpr (PREC == KH_Q4K)
            rh = ld16(W, tid < BN ? (unsigned)(n0 + tid) * (unsigned)(K / QK_K) * Q4K_BYTES +
                                        (unsigned)(k0 / QK_K) * Q4K_BYTES
                                  : OOB);
#pragma unroll
        for (int u = 0; u < B_PT; u++) {
            const int kc = (tid + u * THREADS) & 7;
            rb[u] = ld16(X, brow[u] >= 0 && k0 + 16 * kc < K ? (unsigned)brow[u] * (unsigned)K + (unsigned)(k0 + 16 * kc)
                                                            : OOB);
        }
        if constexpr (PREC != KH_Q4K) {
#pragma unroll
            for (int u = 0; u < WS_PT; u++) {
                const int c = tid + u * THREADS;
                const int row = c / NBS, blk = c % NBS;
                rws[u] = ldf(WS, c < BN * NBS && k0 / BLOCK + blk < nb
                                     ? ((unsigned)(n0 + row) * (unsigned)nb + (unsigned)(k0 / BLOCK + blk)) * 4u
                                     : OOB);
            }
        }
#pragma unroll
        for (int u = 0; u < XS_PT; u++) {
            const int blk = (tid + u * THREADS) % NBS;
            const bool ok = srow[u] >= 0 && k0 / BLOCK + blk < nb;
            const unsigned off = ok ? ((unsigned)srow[u] * (unsigned)nb + (unsigned)(k0 / BLOCK + blk)) * 4u : OOB;
            rxs[u] = ldf(XS, off);
            if constexpr (PREC == KH_Q4K) rxsum[u] = (float)ldi(XSUM, off);
        }
    };

    auto store_stage = [&](int k0) {
#pragma unroll
        for (int u = 0; u < A_PT; u++) {
            const int c = tid + u * THREADS;
            if (c >= A_CH) continue;
            if constexpr (PREC == KH_Q8) {
                const int row = c >> 3, kc = c & 7;
                *reinterpret_cast<int4 *>(sA + row * ASTR + 16 * kc) = ra[u];
            } else if constexpr (PREC == KH_Q4) {
                // byte i of a block: weight i (low nibble), weight 16 + i (high), quant.rs:258-274
                const int row = c / NBS, blk = c % NBS;
                const int4 x = ra[u];
                int4 lo = {nib_minus8(x.x & 0x0f0f0f0f), nib_minus8(x.y & 0x0f0f0f0f), nib_minus8(x.z & 0x0f0f0f0f),
                           nib_minus8(x.w & 0x0f0f0f0f)};
                int4 hi = {nib_minus8((x.x >> 4) & 0x0f0f0f0f), nib_minus8((x.y >> 4) & 0x0f0f0f0f),
                           nib_minus8((x.z >> 4) & 0x0f0f0f0f), nib_minus8((x.w >> 4) & 0x0f0f0f0f)};
                *reinterpret_cast<int4 *>(sA + row * ASTR + 32 * blk) = lo;
                *reinterpret_cast<int4 *>(sA + row * ASTR + 32 * blk + 16) = hi;
            } else {
                // qs byte p of the super-block: sub-block 2(p/32) in the low
                // nibble, 2(p/32)+1 in the high, weight p%32 (mpp.rs:308-313)
                const int row = c / NBS, q = c % NBS;
                const int4 x = ra[u];
                int4 lo = {x.x & 0x0f0f0f0f, x.y & 0x0f0f0f0f, x.z & 0x0f0f0f0f, x.w & 0x0f0f0f0f};
                int4 hi = {(x.x >> 4) & 0x0f0f0f0f, (x.y >> 4) & 0x0f0f0f0f, (x.z >> 4) & 0x0f0f0f0f,
                           (x.w >> 4) & 0x0f0f0f0f};
                const int base = 64 * (q >> 1) + 16 * (q & 1);
                *reinterpret_cast<int4 *>(sA + row * ASTR + base) = lo;
                *reinterpret_cast<int4 *>(sA + row * ASTR + base + 32) = hi;
            }
        }
        if constexpr (PREC == KH_Q4K) {
            if (tid < BN) {
                // 6-bit scales and minimums of the stage's four sub-blocks
                // (scale_min, mpp.rs:276-282)
                const unsigned hb[4] = {(unsigned)rh.x, (unsigned)rh.y, (unsigned)rh.z, (unsigned)rh.w};
                auto byte = [&](int i) { return (hb[i >> 2] >> (8 * (i & 3))) & 0xffu; };  // block byte i
                const float d = half_bits_to_float(hb[0]), dmin = half_bits_to_float(hb[0] >> 16);
                // sub-blocks j = 4 h + jj, h the stage's half of the super-block;
                // each branch indexes the header with constants (a runtime index
                // would put it in scratch memory)
                auto put = [&](int jj, unsigned sc, unsigned mn) {
                    sW[jj][tid] = d * (float)sc;
                    sWm[jj][tid] = dmin * (float)mn;
                };
                if ((k0 % QK_K) / BK == 0) {
#pragma unroll
                    for (int j = 0; j < 4; j++) put(j, byte(4 + j) & 63, byte(8 + j) & 63);
                } else {
#pragma unroll
                    for (int j = 4; j < 8; j++)
                        put(j - 4, (byte(4 + j + 4) & 0xf) | ((byte(4 + j - 4) >> 6) << 4),
                            (byte(4 + j + 4) >> 4) | ((byte(4 + j) >> 6) << 4));
                }
            }
        }
#pragma unroll
        for (int u = 0; u < B_PT; u++) {
            const int c = tid + u * THREADS;
            if (c < B_CH) *reinterpret_cast<int4 *>(sB + (c >> 3) * ASTR + 16 * (c & 7)) = rb[u];
        }
        if constexpr (PREC != KH_Q4K) {
#pragma unroll
            for (int u = 0; u < WS_PT; u++) {
                const int c = tid + u * THREADS;
                if (c < BN * NBS) sW[c % NBS][c / NBS] = rws[u];
            }
        }
#pragma unroll
        for (int u = 0; u < XS_PT; u++) {
            const int c = tid + u * THREADS;
            if (c < BM * NBS) {
                sX[c % NBS][c / NBS] = rxs[u];
                if constexpr (PREC == KH_Q4K) sXs[c % NBS][c / NBS] = rxs[u] * rxsum[u];
            }
        }
    };

    v16f acc[RT][TT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[rt][tt][v] = 0.0f;

    const v16i zero = {};
    const v32f fzero32 = {};
    // One tile's products are held while the next tile's are issued: the
    // matrix core works on tile i while the VALU scales tile i - 1
    // (otherwise every convert waits out its own MFMA).  Tile s of a stage
    // (s = (b RT + rt) TT + tt) keeps its dots in D[s & 1] and its scale
    // products in half h of the pair product P, so nothing is copied
    // between steps; every index is a constant of the unrolled stage (a
    // stage holds an even number of tiles, so the tile pending at a full
    // stage's end is always D[1], half 1).
    v16i D[2] = {};
    v32f P = {};
    bool pending = false;
    auto scale_into = [&](v16f &c, const v32f &pp, int h, const v16i &d) {
#pragma unroll
        for (int v = 0; v < 16; v++) c[v] = __builtin_fmaf(pp[16 * h + v], (float)d[v], c[v]);
    };
    static_assert((NBS * RT * TT) % 2 == 0, "an even number of tiles a stage");
    // split z's stages (all of them without a split)
    int k_begin = 0, k_end = K;
    if (a.ksplit > 1) {
        const int S = (K + BK - 1) / BK, per = (S + a.ksplit - 1) / a.ksplit;
        k_begin = min(S, (int)blockIdx.z * per) * BK;
        k_end = min(K, k_begin + per * BK);
    }
    if (k_begin < k_end) load_stage(k_begin);
    for (int k0 = k_begin; k0 < k_end; k0 += BK) {
        __syncthreads();  // the previous stage's reads of LDS are done
        store_stage(k0);
        __syncthreads();
        if (k0 + BK < k_end) load_stage(k0 + BK);  // in flight during this stage's MFMAs
        const int nblk = min(NBS, (K - k0) / BLOCK);
        // block b's fragments (and its scale columns) from LDS; the next
        // block's are read while this one's products are scaled
        v4i af[2][RT], bf[2][TT];
        // The block's scale products p[r][t] = ws[r] * xs[t] (quant.rs:903;
        // Q4_K: d*sc * xs) are outer products on the matrix core, two 32 x 32
        // tiles per v_mfma_f32_32x32x1_2b_f32 (tile k from lanes 32k..32k+31
        // of both operands, its products in elements 16k..16k+15): the two
        // token tiles of a row tile (TT = 2), else the two row tiles (RT = 2),
        // else two consecutive blocks of the one tile (issued at even blocks).
        constexpr int PR = TT == 2 ? RT : 1;  // pair products per block
        float wa[2][PR], xb[2];
        auto frags = [&](int b, int f) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
                af[f][rt] = *reinterpret_cast<const v4i *>(sA + (wr0 + rt * 32 + (lane & 31)) * ASTR + b * 32 +
                                                           16 * (lane >> 5));
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
                bf[f][tt] = *reinterpret_cast<const v4i *>(sB + (wm0 + tt * 32 + (lane & 31)) * ASTR + b * 32 +
                                                           16 * (lane >> 5));
            if constexpr (TT == 2) {
#pragma unroll
                for (int rt = 0; rt < RT; rt++) wa[f][rt] = sW[b][wr0 + rt * 32 + (lane & 31)];
                xb[f] = sX[b][wm0 + lane];
            } else if constexpr (RT == 2) {
                wa[f][0] = sW[b][wr0 + lane];
                xb[f] = sX[b][wm0 + (lane & 31)];
            } else if ((b & 1) == 0) {  // blocks b and b + 1 (b + 1 < NBS: NBS is even)
                wa[f][0] = sW[b + (lane >> 5)][wr0 + (lane & 31)];
                xb[f] = sX[b + (lane >> 5)][wm0 + (lane & 31)];
            }
        };
        static_assert(NBS % 2 == 0, "block pairs stay within a stage");
        // the half of its pair product that tile (b, rt, tt) takes
        auto half_of = [](int b, int rt, int tt) { return TT == 2 ? tt : RT == 2 ? rt : b & 1; };
        frags(0, 0);
#pragma unroll
        for (int b = 0; b < NBS; b++) {
            if (b >= nblk) {  // a k tail (the last stage only): its last tile is scaled now
                const int sp = b * RT * TT - 1;
                scale_into(acc[RT - 1][TT - 1], P, half_of(b - 1, RT - 1, TT - 1), D[sp & 1]);
                pending = false;
                break;
            }
            const int f = b & 1;
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int tt = 0; tt < TT; tt++) {
                    const int st = (b * RT + rt) * TT + tt;
                    D[st & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[f][rt], bf[f][tt], zero, 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    if (rt == 0 && tt == 0 && b + 1 < NBS && b + 1 < nblk) frags(b + 1, f ^ 1);
                    // the previous tile: (rt, tt - 1), (rt - 1, TT - 1), or the last block's last
                    const int sp = (st + 1) & 1;
                    if (tt > 0) scale_into(acc[rt][tt - 1], P, half_of(b, rt, tt - 1), D[sp]);
                    else if (rt > 0) scale_into(acc[rt - 1][TT - 1], P, half_of(b, rt - 1, TT - 1), D[sp]);
                    else if (pending) scale_into(acc[RT - 1][TT - 1], P, half_of(b - 1, RT - 1, TT - 1), D[sp]);
                    // a pair's product is issued at its first tile, once the
                    // previous pair's last half is used (one pair live at a time)
                    if (half_of(b, rt, tt) == 0) {
                        const float wv = TT == 2 ? wa[f][rt] : wa[f][0];
                        P = __builtin_amdgcn_mfma_f32_32x32x1f32(wv, xb[f], fzero32, 0, 0, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    pending = true;
                }
            if constexpr (PREC == KH_Q4K) {
                // the minimum terms, sum_b dmin*m[r,b] * xs[t,b]*sum[t,b], are a
                // product over blocks: two blocks per 32x32x2 product, straight
                // into the accumulators (mpp.rs:304-315: w = d*sc*q - dmin*m)
                if (b & 1) {
                    const int bb = b - 1 + (lane >> 5);
                    float ma[RT], sb[TT];
#pragma unroll
                    for (int rt = 0; rt < RT; rt++) ma[rt] = -sWm[bb][wr0 + rt * 32 + (lane & 31)];
#pragma unroll
                    for (int tt = 0; tt < TT; tt++) sb[tt] = sXs[bb][wm0 + tt * 32 + (lane & 31)];
#pragma unroll
                    for (int rt = 0; rt < RT; rt++)
#pragma unroll
                        for (int tt = 0; tt < TT; tt++)
                            acc[rt][tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(ma[rt], sb[tt], acc[rt][tt], 0, 0, 0);
                }
            }
        }
    }
    if (pending) scale_into(acc[RT - 1][TT - 1], P, 1, D[1]);
    if (a.ksplit > 1) store_partials<RT, TT>(a, acc, n0 + wr0, m0 + wm0, m_end, lane);
    else store_tiles<RT, TT>(a, acc, n0 + wr0, m0 + wm0, m_end, lane);
}

// ---------------------------------------------------------------------------
// f32 GEMM: v_mfma_f32_32x32x2_f32
// ---------------------------------------------------------------------------

constexpr int FK = 32;          // k per stage (floats)
constexpr int FSTR = FK + 4;    // LDS row stride, floats

template <int WR, int WT, int RT, int TT>
__global__ __launch_bounds__(THREADS) void gemm_f32_kernel(GemmArgs a) {
    constexpr int BN = WR * RT * 32, BM = WT * TT * 32;
    constexpr int A_CH = BN * (FK / 4), B_CH = BM * (FK / 4);
    constexpr int A_PT = (A_CH + THREADS - 1) / THREADS, B_PT = (B_CH + THREADS - 1) / THREADS;
    __shared__ __align__(16) float sA[BN * FSTR];
    __shared__ __align__(16) float sB[BM * FSTR];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr0 = (wave / WT) * RT * 32, wm0 = (wave % WT) * TT * 32;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int K = a.K;
    const rsrc_t W = rsrc(a.w, (size_t)a.N * K * 4);
    const rsrc_t X = rsrc(a.xf, (size_t)a.M * K * 4);

    int4 ra[A_PT], rb[B_PT];
    auto load_stage = [&](int k0) {
#pragma unroll
        for (int u = 0; u < A_PT; u++) {
            const int c = tid + u * THREADS, row = c / (FK / 4), kc = c % (FK / 4);
            ra[u] = c < A_CH && k0 + 4 * kc < K ? ld16(W, ((unsigned)(n0 + row) * (unsigned)K + (unsigned)(k0 + 4 * kc)) * 4u)
                                                 : int4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < B_PT; u++) {
            const int c = tid + u * THREADS, tok = c / (FK / 4), kc = c % (FK / 4);
            rb[u] = c < B_CH && k0 + 4 * kc < K ? ld16(X, ((unsigned)(m0 + tok) * (unsigned)K + (unsigned)(k0 + 4 * kc)) * 4u)
                                                 : int4{0, 0, 0, 0};
        }
    };
    auto store_stage = [&]() {
#pragma unroll
        for (int u = 0; u < A_PT; u++) {
            const int c = tid + u * THREADS;
            if (c < A_CH) *reinterpret_cast<int4 *>(sA + (c / (FK / 4)) * FSTR + 4 * (c % (FK / 4))) = ra[u];
        }
#pragma unroll
        for (int u = 0; u < B_PT; u++) {
            const int c = tid + u * THREADS;
            if (c < B_CH) *reinterpret_cast<int4 *>(sB + (c / (FK / 4)) * FSTR + 4 * (c % (FK / 4))) = rb[u];
        }
    };

    v16f acc[RT][TT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[rt][tt][v] = 0.0f;

    load_stage(0);
    for (int k0 = 0; k0 < K; k0 += FK) {
        __syncthreads();
        store_stage();
        __syncthreads();
        if (k0 + FK < K) load_stage(k0 + FK);
        // lane half h takes k = 16h + 4q + e of the stage; A and B agree on it
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float4 af[RT], bf[TT];
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
                af[rt] = *reinterpret_cast<const float4 *>(sA + (wr0 + rt * 32 + (lane & 31)) * FSTR +
                                                           16 * (lane >> 5) + 4 * q);
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
                bf[tt] = *reinterpret_cast<const float4 *>(sB + (wm0 + tt * 32 + (lane & 31)) * FSTR +
                                                           16 * (lane >> 5) + 4 * q);
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int tt = 0; tt < TT; tt++) {
                    acc[rt][tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[rt].x, bf[tt].x, acc[rt][tt], 0, 0, 0);
                    acc[rt][tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[rt].y, bf[tt].y, acc[rt][tt], 0, 0, 0);
                    acc[rt][tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[rt].z, bf[tt].z, acc[rt][tt], 0, 0, 0);
                    acc[rt][tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[rt].w, bf[tt].w, acc[rt][tt], 0, 0, 0);
                }
        }
    }
    store_tiles<RT, TT>(a, acc, n0 + wr0, m0 + wm0, a.M, lane);
}

// Tile shape for a problem: the largest tile that still gives every CU a
// workgroup, else the smallest.
enum Shape { T128x128, T128x64, T128x32, T64x64 };

Shape pick_shape(int M, int N, int cu) {
    const int forced = env_int("KVAD_GEMM_TILE_M", 0);  // tuning knob: tokens per tile (6464: 64 x 64)
    if (forced == 6464) return T64x64;
    if (forced == 128 || forced == 64 || forced == 32) return forced == 128 ? T128x128 : forced == 64 ? T128x64 : T128x32;
    const long long nt = (N + 127) / 128;
    // 128 x 128 tiles while they give four workgroups per CU; below that,
    // from 128 tokens, 64 x 64 tiles while they give one per two CUs (more,
    // smaller workgroups hide the k-stages' load latency: (512, 896, 4864)
    // 31.0 -> 28.3 us, (1024, 896, 4864) 45.0 -> 41.2, (512, 2048, 1408)
    // 32.6 -> 31.0; at (2048, 4096, 14336) they lose, 461 -> 597, and at 16
    // tokens over 14336x4096 29 -> 45 against 32-token tiles split over k)
    // Token tiles no wider than the tokens need: a tall matrix at 16 or 32
    // tokens (a vocabulary head) gives enough workgroups with 32-token
    // tiles, and 128-token ones would leave three quarters of every tile idle.
    if (M > 64 && nt * ((M + 127) / 128) >= 4LL * cu) return T128x128;
    if (M >= 128 && (long long)((N + 63) / 64) * ((M + 63) / 64) >= cu / 2) return T64x64;
    if (M > 64 && nt * ((M + 127) / 128) >= cu) return T128x128;
    if (M > 32 && nt * ((M + 63) / 64) >= cu) return T128x64;
    return T128x32;
}

}  // namespace

int gemm_tiles(kh_ctx *ctx, int M, int N, int *tile_n) {
    const Shape sh = pick_shape(M, N, ctx->cu_count > 0 ? ctx->cu_count : 256);
    *tile_n = sh == T64x64 ? 64 : 128;
    return sh == T128x128 ? 128 : sh == T128x32 ? 32 : 64;
}

namespace {

template <int PREC>
int launch_i8(kh_ctx *ctx, const GemmArgs &a, int max_tiles, int tile_m, int tile_n) {
    const unsigned gx = (unsigned)((a.N + tile_n - 1) / tile_n) * (a.y2 ? 2u : 1u);
    const unsigned gy = a.tiles ? (unsigned)max_tiles : (unsigned)((a.M + tile_m - 1) / tile_m);
    if (gy == 0) return KH_OK;
    const dim3 grid(gx, gy, a.ksplit > 1 ? (unsigned)a.ksplit : 1u);
    if (tile_n == 64) {
        if (tile_m != 64 || a.tiles) return fail(KH_EINVAL, "gemm: 64-row tiles are 64 tokens wide and ungrouped");
        hipLaunchKernelGGL((gemm_i8_kernel<PREC, 2, 2, 1, 1>), grid, dim3(THREADS), 0, ctx->stream, a);
    } else switch (tile_m) {
        case 128:
            hipLaunchKernelGGL((gemm_i8_kernel<PREC, 2, 2, 2, 2>), grid, dim3(THREADS), 0, ctx->stream, a);
            break;
        case 64:
            hipLaunchKernelGGL((gemm_i8_kernel<PREC, 2, 2, 2, 1>), grid, dim3(THREADS), 0, ctx->stream, a);
            break;
        default:
            hipLaunchKernelGGL((gemm_i8_kernel<PREC, 4, 1, 1, 1>), grid, dim3(THREADS), 0, ctx->stream, a);
            break;
    }
    KH_HIP(hipGetLastError());
    if (a.ksplit > 1) {
        const size_t quads = ((size_t)a.M * a.N + 3) / 4;
        hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, ctx->stream,
                           a.part, a.ksplit, a.M, a.N, a.bias, a.accumulate, a.y);
        KH_HIP(hipGetLastError());
        if (a.y2) {  // the second weight's splits, in the plane after the first's
            hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0,
                               ctx->stream, a.part + (size_t)a.ksplit * a.M * a.N, a.ksplit, a.M, a.N, a.bias,
                               a.accumulate, a.y2);
            KH_HIP(hipGetLastError());
        }
    }
    return KH_OK;
}

// The f32 GEMM runs best on shorter token tiles than the int8 one (swept at
// both prefill shapes): 64 tokens while that still gives two workgroups per
// CU, else 32.
Shape pick_shape_f32(int M, int N, int cu) {
    const int forced = env_int("KVAD_GEMM_TILE_M", 0);
    if (forced == 128 || forced == 64 || forced == 32) return forced == 128 ? T128x128 : forced == 64 ? T128x64 : T128x32;
    const long long nt = (N + 127) / 128;
    return nt * ((M + 63) / 64) >= 2LL * cu ? T128x64 : T128x32;
}

int launch_f32gemm(kh_ctx *ctx, const GemmArgs &a) {
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const unsigned gx = (unsigned)((a.N + 127) / 128);
    switch (pick_shape_f32(a.M, a.N, cu)) {
        case T128x128:
            hipLaunchKernelGGL((gemm_f32_kernel<2, 2, 2, 2>), dim3(gx, (a.M + 127) / 128), dim3(THREADS), 0,
                               ctx->stream, a);
            break;
        case T128x64:
            hipLaunchKernelGGL((gemm_f32_kernel<2, 2, 2, 1>), dim3(gx, (a.M + 63) / 64), dim3(THREADS), 0,
                               ctx->stream, a);
            break;
        default:
            hipLaunchKernelGGL((gemm_f32_kernel<4, 1, 1, 1>), dim3(gx, (a.M + 31) / 32), dim3(THREADS), 0,
                               ctx->stream, a);
            break;
    }
    KH_HIP(hipGetLastError());
    return KH_OK;
}

// Row-at-a-time path for shapes the tiled kernels do not take (f32 weights
// whose width is not a multiple of 4): one GEMV job per activation row.
int matmul_rows(kh_ctx *ctx, const kh_weight *w, const float *xs, size_t m, const float *bias, float *y,
                int accumulate) {
    std::vector<GemvJob> jobs(m);
    for (size_t i = 0; i < m; i++) {
        GemvJob &j = jobs[i];
        j = GemvJob{};
        j.w = w->qs;
        j.xf = xs + i * w->cols;
        j.bias = bias;
        j.y = y + i * w->rows;
        j.rows = (int)w->rows;
        j.cols = (int)w->cols;
        j.accumulate = accumulate;
    }
    return launch_gemv(ctx, w->precision, jobs.data(), (int)m);
}

}  // namespace

namespace {
// KVAD_MATMUL_GEMM=1 sends every m > 1 to the MFMA GEMM (for comparisons).
bool matmul_force_gemm() { return env_int("KVAD_MATMUL_GEMM", 0) == 1; }
}  // namespace

namespace {
// The split-K workspace: one fixed allocation for the partials, made on the
// first split launch and never moved, so graphs captured over later launches
// stay valid; a split whose partials do not fit is cut to what fits.
constexpr size_t SPLIT_BYTES = 64u << 20;
const int SPLIT_MIN_STAGES = env_int("KVAD_GEMM_SPLIT_MIN", 2);  // tuning knobs
const int SPLIT_MAX = env_int("KVAD_GEMM_SPLIT_MAX", 32);
const int SPLIT_PER_CU = env_int("KVAD_GEMM_SPLIT_PER_CU", 2);
}  // namespace

int gemm_split_reserve(kh_ctx *ctx) {
    if (ctx->gemm.ptr) return KH_OK;
    KH_HIP(hipMalloc(&ctx->gemm.ptr, SPLIT_BYTES));
    ctx->gemm.bytes = SPLIT_BYTES;
    return KH_OK;
}

int plan_split(kh_ctx *ctx, GemmArgs &a, int tile_m, int tile_n) {
    a.ksplit = 0;
    if (a.tiles) return KH_OK;  // grouped launches are not split
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    // Split the k-stages so that the grid comes to about SPLIT_PER_CU
    // workgroups per CU (a CU holds several: one's loads wait while
    // another's MFMAs run), with at least SPLIT_MIN_STAGES stages a split,
    // at most SPLIT_MAX splits, and partials (4 M N bytes a split, written
    // and read again) of at most the weights' N K bytes or 4 MiB, whichever
    // is more (a small weight such as a router's 64 rows would otherwise
    // never split: 512 tokens x 64 x 2048, 16 workgroups, 22.6 us unsplit).
    // a paired launch (a.y2) holds both weights' tiles and partial planes
    const int pair = a.y2 ? 2 : 1;
    const long long tiles = (long long)((a.N + tile_n - 1) / tile_n) * ((a.M + tile_m - 1) / tile_m) * pair;
    const int S = (a.K + BK - 1) / BK;
    const size_t plane = (size_t)a.M * a.N * 4 * pair;
    long long ks = ((long long)SPLIT_PER_CU * cu + tiles / 2) / tiles;
    ks = std::min<long long>(ks, S / SPLIT_MIN_STAGES);
    ks = std::min<long long>(ks, SPLIT_MAX);
    ks = std::min<long long>(ks, (long long)(std::max((size_t)a.N * a.K * pair, (size_t)4 << 20) / plane));
    const int forced = env_int("KVAD_GEMM_KSPLIT", 0);  // tuning knob: k splits (1: none)
    if (forced > 0) ks = std::min(forced, S);
    ks = std::min<long long>(ks, (long long)(SPLIT_BYTES / plane));
    if (ks < 2) return KH_OK;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    KH_HIP(hipStreamIsCapturing(ctx->stream, &cap));
    if (cap == hipStreamCaptureStatusNone) {  // no allocation under capture
        const int rc = gemm_split_reserve(ctx);
        if (rc) return rc;
    }
    if (!ctx->gemm.ptr) return KH_OK;
    a.ksplit = (int)ks;
    a.part = static_cast<float *>(ctx->gemm.ptr);
    return KH_OK;
}

int launch_matmul(kh_ctx *ctx, const kh_weight *w, const float *xs, size_t m, const float *bias, float *y,
                  int accumulate) {
    const size_t rows = w->rows, cols = w->cols;
    // 32-bit buffer offsets: the weights and activations (plus one tile of
    // overhang) must stay below 4 GiB
    const size_t wb = w->precision == KH_F32 ? 4 * rows * cols : rows * cols;
    const size_t xb = w->precision == KH_F32 ? 4 * m * cols : m * cols;
    if (wb + 4 * 128 * cols >= 0xffffffffull || xb + 4 * 128 * cols >= 0xffffffffull || rows > 0x7fffffff ||
        m > 0x7fffffff)
        return fail(KH_DECLINED, "matmul: operands of 4 GiB or more are not addressed here");
    GemmArgs a{};
    a.w = w->qs;
    a.ws = w->scales;
    a.bias = bias;
    a.y = y;
    a.accumulate = accumulate;
    a.M = (int)m;
    a.N = (int)rows;
    a.K = (int)cols;
    if (w->precision == KH_F32) {
        if (cols % 4) return matmul_rows(ctx, w, xs, m, bias, y, accumulate);
        a.xf = xs;
        return launch_f32gemm(ctx, a);
    }
    // up to eight rows: the multi-token GEMV quantises them as it stages them
    // (QActBatch::new's codes, one launch fewer) while they are few values
    const bool multi = matmul_takes_multi(m, rows, cols) && !matmul_force_gemm();
    if (multi && multi_stages_f32(w->precision, m, cols))
        return launch_gemv_multi_jobs(ctx, 1, &w, &bias, &y, &accumulate, QAct{}, m, xs);
    // QActBatch::new (quant.rs:693-714): the activation rows quantised per block
    const size_t qb = (m * cols + 255) / 256 * 256, sb = (4 * m * cols / BLOCK + 255) / 256 * 256;
    int rc = ensure(ctx, ctx->ws, qb + 2 * sb);
    if (rc) return rc;
    char *p = static_cast<char *>(ctx->ws.ptr);
    QAct q{reinterpret_cast<int8_t *>(p), reinterpret_cast<float *>(p + qb), reinterpret_cast<int32_t *>(p + qb + sb)};
    if ((rc = launch_qact(ctx, xs, m, cols, q))) return rc;
    return launch_matmul_q(ctx, w, q, m, bias, y, accumulate);
}

int launch_matmul_q(kh_ctx *ctx, const kh_weight *w, const QAct &q, size_t m, const float *bias, float *y,
                    int accumulate) {
    const size_t rows = w->rows, cols = w->cols;
    if (w->precision == KH_F32) return fail(KH_EINVAL, "matmul: f32 weights take f32 rows");
    if (rows * cols + 4 * 128 * cols >= 0xffffffffull || m * cols + 4 * 128 * cols >= 0xffffffffull ||
        rows > 0x7fffffff || m > 0x7fffffff)
        return fail(KH_DECLINED, "matmul: operands of 4 GiB or more are not addressed here");
    // a few tokens: stream the weights once through the multi-token GEMV
    if (matmul_takes_multi(m, rows, cols) && !matmul_force_gemm())
        return launch_gemv_multi_jobs(ctx, 1, &w, &bias, &y, &accumulate, q, m);
    GemmArgs a{};
    a.w = w->qs;
    a.ws = w->scales;
    a.bias = bias;
    a.y = y;
    a.accumulate = accumulate;
    a.M = (int)m;
    a.N = (int)rows;
    a.K = (int)cols;
    a.xq = q.qs;
    a.xs = q.scales;
    a.xsum = q.sums;
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const Shape sh = pick_shape(a.M, a.N, cu);
    const int tile_m = sh == T128x128 ? 128 : sh == T128x32 ? 32 : 64, tile_n = sh == T64x64 ? 64 : 128;
    int rc = plan_split(ctx, a, tile_m, tile_n);
    if (rc) return rc;
    return launch_gemm_q(ctx, w->precision, a, 0, tile_m, tile_n);
}

int launch_gemm_q(kh_ctx *ctx, int precision, const GemmArgs &a, int max_tiles, int tile_m, int tile_n) {
    if (a.tiles && (!a.wtab || !a.wstab)) return fail(KH_EINVAL, "gemm: grouped launch without weight tables");
    switch (precision) {
        case KH_Q8: return launch_i8<KH_Q8>(ctx, a, max_tiles, tile_m, tile_n);
        case KH_Q4: return launch_i8<KH_Q4>(ctx, a, max_tiles, tile_m, tile_n);
        case KH_Q4K: return launch_i8<KH_Q4K>(ctx, a, max_tiles, tile_m, tile_n);
        default: return fail(KH_EINVAL, "gemm: the grouped kernel takes quantised weights");
    }
}

}  // namespace kh
