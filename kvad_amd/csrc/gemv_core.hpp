// The building blocks of the quantised GEMV kernels (gemv.hip):
// job tables, the 16-byte weight chunks a lane loads and their block dots
// (Weight::qrow, crates/llm/src/quant.rs:410-452; q4_row_dots, quant.rs:168-189;
// Q4_K, crates/gpu/src/mpp.rs:241-315), and the staging of the activation in
// LDS with its quantisation (QActivation::new, quant.rs:1044-1066).
#pragma once

#include "common.hpp"
#include "device.hpp"

namespace kh {
namespace {

using namespace dev;

constexpr int WAVES_PER_BLOCK = 4;
constexpr int MAX_JOBS = 24;

struct JobTable {
    // the launch's n jobs; first[i] is job i's first workgroup, ascending,
    // INT_MAX past the n jobs, so a workgroup finds its job from one batch
    // of scalar loads
    int n;
    int first[MAX_JOBS];
    GemvJob j[MAX_JOBS];
    // ROUTE kernels: 1 + the job whose one workgroup, having computed a
    // token's router logits, also routes them (route.hpp); 0: none
    int route_job;
    RouteArgs route;
    // 1 + the job whose workgroups also keep the greedy choice over their
    // rows r >= 1 (the largest, the lowest index on ties, NaN never):
    // workgroup g writes arg_v[g], arg_i[g] and workgroup 0 the count to
    // *arg_n; 0: none
    int arg_job, arg_cap;
    float *arg_v;
    int *arg_i, *arg_n;
    GreedyTail tail;  // tail.arrivals set: the step ends in this launch
};

// The job of workgroup `blk`: the last job whose first workgroup is at or
// before it (jobs without workgroups start where the next one does).  v - blk
// - 1 has its sign bit set exactly when v <= blk (v, blk < 2^31), a count in
// scalar registers.  Jobs 1..8 come packed as 16-bit words in the kernel's
// first four arguments, which are preloaded into scalar registers; jobs 9..
// are looked up in the table by workgroups past job 8 only.
struct Firsts {
    unsigned f[4];
};
__device__ __forceinline__ int at_or_before(unsigned v, int blk) { return (int)((v - (unsigned)blk - 1u) >> 31); }
__device__ __forceinline__ int job_of(const JobTable &tab, const Firsts &fp, int blk) {
    int ji = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) ji += at_or_before(fp.f[k] & 0xffffu, blk) + at_or_before(fp.f[k] >> 16, blk);
    if (ji == 8) {
#pragma unroll
        for (int i = 9; i < MAX_JOBS; i++) ji += at_or_before((unsigned)tab.first[i], blk);
    }
    return ji;
}
// The same from the table alone (one batch of scalar loads for jobs 1..16).
__device__ __forceinline__ int job_of(const JobTable &tab, int blk) {
    int ji = 0;
#pragma unroll
    for (int i = 1; i <= 16; i++) ji += at_or_before((unsigned)tab.first[i], blk);
    if (ji == 16) {
#pragma unroll
        for (int i = 17; i < MAX_JOBS; i++) ji += at_or_before((unsigned)tab.first[i], blk);
    }
    return ji;
}

// The job table's workgroup index, once every job's wave0 is set; and jobs
// 1..8 of it packed for the kernel's arguments (launches have fewer than
// 0xffff workgroups).
inline void set_first(JobTable &tab) {
    for (int i = 0; i < MAX_JOBS; i++) tab.first[i] = i < tab.n ? tab.j[i].wave0 : 0x7fffffff;
}
// Job 0's fields for the kernel's preloaded arguments (see gemv_kernel).
struct Lead {
    const void *w;
    const float *ws, *xf, *x2;
    int rows;
    unsigned colsnw;  // cols | nwaves << 16; bit 30: every job stages job 0's input; bit 31: job 0 from the table
};
inline Lead lead_job(const JobTable &tab) {
    const GemvJob &j = tab.j[0];
    const bool slow = j.wtab || j.cols > 0xffff || j.nwaves > 0x3fff;
    bool shared = j.xf != nullptr;  // an f32 input (codes made elsewhere come from the table)
    for (int i = 1; i < tab.n && shared; i++) {
        const GemvJob &o = tab.j[i];
        shared = o.xf == j.xf && o.xf2 == j.xf2 && o.norm_w == j.norm_w && o.cols == j.cols;
    }
    return {j.w, j.ws, j.xf, j.xf2 ? j.xf2 : j.norm_w, j.rows,
            slow ? 1u << 31 : (unsigned)j.cols | (unsigned)j.nwaves << 16 | (shared ? 1u << 30 : 0u)};
}
inline Firsts packed_first(const JobTable &tab) {
    Firsts fp;
    for (int k = 0; k < 4; k++) {
        const unsigned lo = (unsigned)(tab.first[2 * k + 1] < 0xffff ? tab.first[2 * k + 1] : 0xffff);
        const unsigned hi = (unsigned)(tab.first[2 * k + 2] < 0xffff ? tab.first[2 * k + 2] : 0xffff);
        fp.f[k] = lo | hi << 16;
    }
    return fp;
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

__host__ __device__ inline int align16(int n) { return (n + 15) & ~15; }

// silu(g) * u with silu(g) = g / (1 + exp(-g)), as swiglu_inplace computes
// it (tensor.rs:344-350): one divide, one product.
__device__ __forceinline__ float swiglu1(float g, float u) {
    const float silu = g / (1.0f + expf(-g));
    return silu * u;
}

// ---------------------------------------------------------------------------
// activation quantisation: 8 lanes per 32-block, 4 values each
// ---------------------------------------------------------------------------

// The block's scale amax / 127 and its inverse (quant.rs:1052-1053), each
// rounded once as IEEE division rounds them, in a third of the instructions
// of two divides:
//  - amax / 127: the product with RN(1/127) corrected once by its exact
//    residual amax - 127 q (Markstein's division step, P. Markstein, IBM J.
//    Res. Dev. 34(1), 1990);
//  - 1 / scale: v_rcp_f32 (within an ulp) and one Markstein step.
// Both equal the IEEE results for every finite amax >= 0 whose scale is zero
// or normal (kh_debug_quant_check scans all 2^32 floats); an infinite amax,
// or a scale that underflows to a subnormal, takes the divides.
__device__ __forceinline__ void qscale(float amax, float &scale, float &inv) {
    constexpr float r = 0x1.020408p-7f;  // RN(1/127)
    const float q = amax * r;
    const float rem = __builtin_fmaf(-q, 127.0f, amax);
    scale = __builtin_fmaf(rem, r, q);
    // +0 or +normal (v_cmp_class: bit 6 = +0, bit 8 = +normal)
    if (__builtin_expect(__builtin_amdgcn_classf(scale, (1 << 6) | (1 << 8)), 1)) {
        const float y = __builtin_amdgcn_rcpf(scale);
        const float e = __builtin_fmaf(-scale, y, 1.0f);
        inv = scale > 0.0f ? __builtin_fmaf(e, y, y) : 0.0f;
    } else {
        scale = amax / 127.0f;
        inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    }
}

// (t.round().clamp(-127.0, 127.0) as i8) of quant.rs:1059: half away from
// zero as trunc(t + copysign(0.5 - 2^-25, t)) (the sum rounds up to the next
// integer exactly when t's fraction is at least a half), the clamp on the
// integer; NaN gives 0 and +-inf +-127, as Rust's saturating cast does.
// Equal to the definition for all 2^32 floats (kh_debug_quant_check).
__device__ __forceinline__ int qround(float t) {
    const int q = (int)(t + __builtin_copysignf(0x1.fffffep-2f, t));
    return min(max(q, -127), 127);
}

// One lane's share of QActivation::new (quant.rs:1051-1064): returns the four
// codes packed; *scale and *sum are the block's (same in all 8 lanes).
__device__ __forceinline__ int quantize4(float4 v, float *scale_out, int *sum_out) {
    // the block's amax over its 8 lanes; NaN is passed over, as f32::max does
    // (fmax with 0 also maps a lane of four NaN to 0), and the non-negative
    // values compare as their bit patterns do, so the lanes meet with
    // integer maxima
    const float a4 = fmaxf(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))), 0.0f);
    int ab = __builtin_bit_cast(int, a4);
    ab = max(ab, dpp<DPP_XOR1>(ab));
    ab = max(ab, dpp<DPP_XOR2>(ab));
    ab = max(ab, dpp<DPP_HALF_MIRROR>(ab));
    float scale, inv;
    qscale(__builtin_bit_cast(float, ab), scale, inv);
    const int q0 = qround(v.x * inv), q1 = qround(v.y * inv), q2 = qround(v.z * inv), q3 = qround(v.w * inv);
    // bytes q0 q1 q2 q3, low to high
    const unsigned p01 = __builtin_amdgcn_perm((unsigned)q1, (unsigned)q0, 0x0c0c0400u);
    const unsigned p23 = __builtin_amdgcn_perm((unsigned)q3, (unsigned)q2, 0x0c0c0400u);
    const int packed = (int)(p01 | (p23 << 16));
    int s = (q0 + q1) + (q2 + q3);
    s += dpp<DPP_XOR1>(s);
    s += dpp<DPP_XOR2>(s);
    s += dpp<DPP_HALF_MIRROR>(s);
    *scale_out = scale;
    *sum_out = s;
    return packed;
}

// ---------------------------------------------------------------------------
// the quantised GEMV kernel family
// ---------------------------------------------------------------------------

constexpr int WPB = 8;  // waves per workgroup (512 threads)

// Activation blocks the LDS stage holds for a launch whose widest row has
// `C` chunks at `cpl` chunks per lane per segment: the row's blocks, padded
// with zero blocks up to what the last segment's lanes index.
__host__ __device__ inline int padded_blocks(int prec, int C, int cpl) {
    const int nseg = (C + WAVE * cpl - 1) / (WAVE * cpl);
    const int cp = nseg * WAVE * cpl;
    return prec == KH_Q8 ? cp / 2 : cp;
}

// A row group's weight chunks in registers.
template <int PREC, int CPL, int R>
struct Chunks {
    int4 w[R][CPL];
    int4 h[R][CPL];      // Q4_K block headers
    float s[R][CPL];     // q8/q4 block scales
};

// PAIR: rows r0 + i alternate between two weights (W, WS for even i, W2,
// WS2 for odd), row (r0 + i) / 2 of each (r0 is even).
template <int PREC, int CPL, int R, bool PAIR = false>
__device__ __forceinline__ void load_chunks(Chunks<PREC, CPL, R> &c, const rsrc_t &W1, const rsrc_t &WS1, int r0,
                                            int cols, int nb, int seg, int lane, const rsrc_t &W2,
                                            const rsrc_t &WS2) {
    // Offsets are a row's part, the same in every lane (made scalar with
    // readfirstlane, so the compiler cannot fold it into a per-lane multiply),
    // plus the lane's part, the same at every step.  The whole offset stays
    // in the vector operand, which the buffer's range check covers.
#pragma unroll
    for (int i = 0; i < R; i++) {
        const unsigned r = PAIR ? (unsigned)((r0 + i) >> 1) : (unsigned)(r0 + i);
        const rsrc_t &W = PAIR && (i & 1) ? W2 : W1;
        const rsrc_t &WS = PAIR && (i & 1) ? WS2 : WS1;
        if constexpr (PREC == KH_Q8) {
            // chunk gl = seg * 64 * CPL + lane: weights 16 gl.., block gl / 2
            const unsigned uw = __builtin_amdgcn_readfirstlane(r * (unsigned)cols + (unsigned)(seg * CPL) * 1024u);
            const unsigned us = __builtin_amdgcn_readfirstlane(r * (unsigned)nb * 4u + (unsigned)(seg * CPL) * 128u);
            const unsigned wo = uw + (unsigned)lane * 16u, so = us + (unsigned)(lane >> 1) * 4u;
#pragma unroll
            for (int t = 0; t < CPL; t++) {
                c.w[i][t] = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(W, wo, t * 1024, 0));
                c.s[i][t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(WS, so, t * 128, 0));
            }
        } else if constexpr (PREC == KH_Q4) {
            const unsigned uw = __builtin_amdgcn_readfirstlane(r * (unsigned)(cols / 2) + (unsigned)(seg * CPL) * 1024u);
            const unsigned us = __builtin_amdgcn_readfirstlane(r * (unsigned)nb * 4u + (unsigned)(seg * CPL) * 256u);
            const unsigned wo = uw + (unsigned)lane * 16u, so = us + (unsigned)lane * 4u;
#pragma unroll
            for (int t = 0; t < CPL; t++) {
                c.w[i][t] = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(W, wo, t * 1024, 0));
                c.s[i][t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(WS, so, t * 256, 0));
            }
        } else {
            // chunk gl: block gl / 8 (= seg * 8 * CPL + lane / 8), 16 bytes at
            // 16 + 16 (lane & 7) of it; 64 chunks = 8 blocks = 1152 bytes per t
            const unsigned row_bytes = (unsigned)(cols / QK_K) * Q4K_BYTES;
            const unsigned ub = __builtin_amdgcn_readfirstlane(r * row_bytes + (unsigned)(seg * CPL) * 8u * Q4K_BYTES);
            const unsigned bo = ub + (unsigned)(lane >> 3) * Q4K_BYTES;
            const unsigned wo = bo + 16u + 16u * (unsigned)(lane & 7);
#pragma unroll
            for (int t = 0; t < CPL; t++) {
                c.w[i][t] = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(W, wo, t * 1152, 0));
                c.h[i][t] = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(W, bo, t * 1152, 0));
            }
        }
    }
}

// The 6-bit scale and minimum of Q4_K sub-block j (mpp.rs:276-282) from
// bytes 4..15 of the block header (h.y = bytes 4..7, h.z = 8..11, h.w =
// 12..15, i.e. s[0..3], s[4..7], s[8..11]), with lane constants: j < 4 reads
// s[j] & 63 and s[j+4] & 63; j >= 4 reads the low four bits from s[j+4] and
// the top two from s[j-4] and s[j].  Two selects, four bit-field extracts and
// two shift-ors.
struct Q4kLane {
    bool hi4;           // j >= 4
    unsigned o1, w1;    // scale's low bits: offset and width in hi4 ? h.w : h.y
    unsigned o3;        // minimum's low bits: offset (same width) in hi4 ? h.w : h.z
    unsigned o2, w2;    // top two bits (j >= 4; width 0 otherwise) in h.y / h.z
};
__device__ __forceinline__ Q4kLane q4k_lane(int j) {
    const unsigned jj = (unsigned)(j & 3);
    const bool hi4 = j >= 4;
    return {hi4, 8 * jj, hi4 ? 4u : 6u, hi4 ? 8 * jj + 4 : 8 * jj, 8 * jj + 6, hi4 ? 2u : 0u};
}
__device__ __forceinline__ void q4k_scale_min_bfe(const int4 &h, const Q4kLane &L, unsigned &sc, unsigned &mn) {
    const unsigned y = (unsigned)h.y, z = (unsigned)h.z, w = (unsigned)h.w;
    sc = __builtin_amdgcn_ubfe(L.hi4 ? w : y, L.o1, L.w1) | (__builtin_amdgcn_ubfe(y, L.o2, L.w2) << 4);
    mn = __builtin_amdgcn_ubfe(L.hi4 ? w : z, L.o3, L.w1) | (__builtin_amdgcn_ubfe(z, L.o2, L.w2) << 4);
}

// The chunks' contribution to each row's accumulator, in chunk order.
template <int PREC, int CPL, int R, bool DOTS>
__device__ __forceinline__ void compute_chunks(const Chunks<PREC, CPL, R> &c, float (&acc)[R], const int8_t *sq,
                                               const float *ssc, const int *ssum, int seg, int lane, int r0,
                                               int rows, int nb, int C, int32_t *dots) {
    const int gl = seg * WAVE * CPL + lane;
    if constexpr (PREC == KH_Q8) {
#pragma unroll
        for (int t = 0; t < CPL; t++) {
            const int g = gl + t * WAVE;
            const int4 a = *reinterpret_cast<const int4 *>(sq + g * 16);
            const float as = ssc[g >> 1];
#pragma unroll
            for (int i = 0; i < R; i++) {
                int d = dot4(c.w[i][t].x, a.x, 0);
                d = dot4(c.w[i][t].y, a.y, d);
                d = dot4(c.w[i][t].z, a.z, d);
                d = dot4(c.w[i][t].w, a.w, d);
                d += dpp<DPP_XOR1>(d);  // the other half of the 32-block
                float s = c.s[i][t] * as;
                s = s * (float)d;
                acc[i] += (lane & 1) ? 0.0f : s;
                if (DOTS && !(lane & 1) && g < C && r0 + i < rows) dots[(size_t)(r0 + i) * nb + (g >> 1)] = d;
            }
        }
    } else if constexpr (PREC == KH_Q4) {
#pragma unroll
        for (int t = 0; t < CPL; t++) {
            const int g = gl + t * WAVE;
            const int4 alo = *reinterpret_cast<const int4 *>(sq + g * 32);
            const int4 ahi = *reinterpret_cast<const int4 *>(sq + g * 32 + 16);
            const float as = ssc[g];
            const int asum = ssum[g];
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int4 q = c.w[i][t];
                int lo = dot4(q.x & 0x0f0f0f0f, alo.x, 0);
                lo = dot4(q.y & 0x0f0f0f0f, alo.y, lo);
                lo = dot4(q.z & 0x0f0f0f0f, alo.z, lo);
                lo = dot4(q.w & 0x0f0f0f0f, alo.w, lo);
                int hi = dot4((q.x >> 4) & 0x0f0f0f0f, ahi.x, 0);
                hi = dot4((q.y >> 4) & 0x0f0f0f0f, ahi.y, hi);
                hi = dot4((q.z >> 4) & 0x0f0f0f0f, ahi.z, hi);
                hi = dot4((q.w >> 4) & 0x0f0f0f0f, ahi.w, hi);
                const int d = lo + hi - 8 * asum;  // quant.rs:187
                float s = c.s[i][t] * as;
                s = s * (float)d;
                acc[i] += s;
                if (DOTS && g < C && r0 + i < rows) dots[(size_t)(r0 + i) * nb + g] = d;
            }
        }
    } else {
        // Q4_K: the sub-block a lane finishes is fixed by the lane (64 % 8 == 0)
        const int half = lane & 1, cc = (lane & 7) >> 1, j = 2 * cc + half;
        const Q4kLane L = q4k_lane(j);
#pragma unroll
        for (int t = 0; t < CPL; t++) {
            const int g = gl + t * WAVE;
            const int b0 = (g >> 3) * 8 + 2 * cc;  // sub-blocks b0 (low nibbles), b0 + 1 (high)
            const int4 alo = *reinterpret_cast<const int4 *>(sq + b0 * 32 + 16 * half);
            const int4 ahi = *reinterpret_cast<const int4 *>(sq + (b0 + 1) * 32 + 16 * half);
            const float as = ssc[b0 + half];
            const int asum = ssum[b0 + half];
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int4 q = c.w[i][t];
                int lo = dot4(q.x & 0x0f0f0f0f, alo.x, 0);
                lo = dot4(q.y & 0x0f0f0f0f, alo.y, lo);
                lo = dot4(q.z & 0x0f0f0f0f, alo.z, lo);
                lo = dot4(q.w & 0x0f0f0f0f, alo.w, lo);
                int hi = dot4((q.x >> 4) & 0x0f0f0f0f, ahi.x, 0);
                hi = dot4((q.y >> 4) & 0x0f0f0f0f, ahi.y, hi);
                hi = dot4((q.z >> 4) & 0x0f0f0f0f, ahi.z, hi);
                hi = dot4((q.w >> 4) & 0x0f0f0f0f, ahi.w, hi);
                lo += dpp<DPP_XOR1>(lo);
                hi += dpp<DPP_XOR1>(hi);
                const int d = half ? hi : lo;
                // 6-bit scale and minimum of sub-block j (mpp.rs:276-282)
                const int4 h = c.h[i][t];
                unsigned sc, mn;
                q4k_scale_min_bfe(h, L, sc, mn);
                // sc * dot (|dot| < 2^16, sc < 64) and mn * asum are exact 24-bit
                // products, and f32(d) * sc is exact, so d * (sc * dot) is the
                // block's d * sc * dot: dmin * mn * asum rounded once, d * sc *
                // dot less that rounded once (one fma, which takes the f16
                // header halves as they are), then one fma into the row
                const int isc = mul24((int)sc, d);
                const int imn = mul24((int)mn, asum);
                const float t2 = __builtin_fmaf(half_bits_to_float((unsigned)h.x >> 16), (float)imn, -0.0f);
                const float s = __builtin_fmaf(half_bits_to_float((unsigned)h.x), (float)isc, -t2);
                acc[i] = __builtin_fmaf(as, s, acc[i]);
                if (DOTS && g < C && r0 + i < rows) dots[(size_t)(r0 + i) * nb + (g >> 3) * 8 + j] = d;
            }
        }
    }
}

// Activation staging.  A thread's activation loads are issued before the
// workgroup's first weight loads: vector loads complete in order, so an
// activation load issued after them would wait for HBM.  The input kind is a
// template parameter so that a launch holds registers only for what it loads.
constexpr int IN_F32 = 0;       // f32 x
constexpr int IN_SWIGLU = 1;    // swiglu(xf, xf2)
constexpr int IN_CODES = 2;     // int8 codes, scales and sums made elsewhere
constexpr int IN_NORM = 3;      // rms_norm(xf) * norm_w

// SB float4s (or code int4s) per thread per batch: 4, or 8 where the
// kernel's weight registers leave room (one batch then covers 16384 columns).
template <int KIND, int SB>
struct Stage {
    float4 v[SB];                    // f32 input, or int4 codes
    float4 u[KIND == IN_F32 ? 1 : SB];  // swiglu's second input, norm weights, or (scale, sum)
};

__device__ __forceinline__ float4 zero4() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// The thread's loads: float4 c = k * T + tid of the f32 input (block c >> 3),
// or int4 c of the codes and scale and sum c.  One such batch covers the
// whole activation (the launcher checks it: stage_fits).
template <int KIND, int SB, int NWV>
__device__ __forceinline__ void stage_load(const GemvJob &job, const float *xf, const float *x2, Stage<KIND, SB> &st,
                                           int nb, int tid) {
    constexpr int T = WAVE * NWV;
    // buffer loads: past the input's end they return zeros, with no branch
    if constexpr (KIND == IN_CODES) {
        const rsrc_t Q = rsrc(job.xq, (size_t)nb * BLOCK), S = rsrc(job.xs, (size_t)nb * 4),
                     M = rsrc(job.xsum, (size_t)nb * 4);
#pragma unroll
        for (int k = 0; k < SB; k++) {
            const unsigned c = (unsigned)(k * T + tid);
            st.v[k] = __builtin_bit_cast(float4, bld16(Q, c * 16));
            st.u[k] = make_float4(bldf(S, c * 4), __builtin_bit_cast(float, bldi(M, c * 4)), 0.f, 0.f);
        }
    } else {
        // x2: swiglu's second input or the norm's weights
        const rsrc_t X = rsrc(xf, (size_t)nb * BLOCK * 4);
        const rsrc_t X2 = rsrc(KIND == IN_F32 ? xf : x2, (size_t)nb * BLOCK * 4);
#pragma unroll
        for (int k = 0; k < SB; k++) {
            const unsigned c = (unsigned)(k * T + tid);
            st.v[k] = __builtin_bit_cast(float4, bld16(X, c * 16));
            if constexpr (KIND != IN_F32) st.u[k] = __builtin_bit_cast(float4, bld16(X2, c * 16));
        }
    }
}

// Stages the activation of `job` in LDS for a workgroup: int8 codes, scales
// and code sums of PB blocks (blocks past nb are zero).  From f32 input it
// quantises as QActivation::new (quant.rs:1044-1066), first applying
// rms_norm (tensor.rs:329-333) for IN_NORM or swiglu(xf, xf2)
// (tensor.rs:344-350) for IN_SWIGLU; codes made elsewhere are copied.  `st` holds batch 0,
// loaded by stage_load.  Every workgroup computes the same values.
template <int KIND, int SB, int NWV>
__device__ __forceinline__ void stage_activation(const GemvJob &job, Stage<KIND, SB> &st, int8_t *sq, float *ssc,
                                                 int *ssum, int PB, int nb, int cols, int tid, int lane, int wv) {
    constexpr int T = WAVE * NWV;
    if constexpr (KIND == IN_CODES) {
#pragma unroll
        for (int k = 0; k < SB; k++) {
            const int c = k * T + tid;
            if (c < PB * 2) reinterpret_cast<int4 *>(sq)[c] = __builtin_bit_cast(int4, st.v[k]);
            if (c < PB) {
                ssc[c] = st.u[k].x;
                ssum[c] = __builtin_bit_cast(int, st.u[k].y);
            }
        }
        return;
    } else {
        constexpr bool nw = KIND == IN_NORM;
        float inv = 1.0f;
        if constexpr (nw) {
            // Sum of squares over the thread's float4s in index order, then
            // over the wave, then over the waves in order: every workgroup
            // gets the same sum.
            __shared__ float s_ss[NWV];
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < SB; k++) {
                const float4 v = st.v[k];
                const float a = v.x * v.x, b = v.y * v.y, c = v.z * v.z, d = v.w * v.w;
                ss = ss + ((a + b) + (c + d));
            }
            ss = wave_sum(ss);
            if (lane == 0) s_ss[wv] = ss;
            __syncthreads();
            float t = 0.0f;
#pragma unroll
            for (int w = 0; w < NWV; w++) t = t + s_ss[w];
            inv = 1.0f / sqrtf(t / (float)cols + job.norm_eps);
        }
#pragma unroll
        for (int k = 0; k < SB; k++) {
            const int i = k * T + tid, b = i >> 3;
            if (b >= PB) break;  // uniform per 8-lane block group, and past every later k
            float4 x = st.v[k];
            if constexpr (nw) {
                const float4 w = st.u[k];  // zeros past the end, like x
                x = make_float4((x.x * inv) * w.x, (x.y * inv) * w.y, (x.z * inv) * w.z, (x.w * inv) * w.w);
            }
            if constexpr (KIND == IN_SWIGLU) {
                const float4 u = st.u[k];
                x = make_float4(swiglu1(x.x, u.x), swiglu1(x.y, u.y), swiglu1(x.z, u.z), swiglu1(x.w, u.w));
            }
            float scale;
            int s;
            const int packed = quantize4(x, &scale, &s);
            reinterpret_cast<int *>(sq)[i] = packed;
            if ((tid & 7) == 0) {
                ssc[b] = scale;
                ssum[b] = s;
            }
        }
    }
}

// Whether one staging batch (SB loads per thread) covers PB blocks.
// A kernel stages 8 loads per thread where its weight registers leave room
// (CPL >= 4) or where it is built WIDE (rows of several segments), else 4.
__host__ __device__ constexpr int stage_batch(int cpl, bool wide) { return cpl >= 4 || wide ? 8 : 4; }
__host__ __device__ inline bool stage_fits(int kind, int PB, int sb, int nwv) {
    const int cap = sb * WAVE * nwv;
    return kind == IN_CODES ? PB * 2 <= cap : PB * 8 <= cap;
}

// The input kind of a job.
__host__ __device__ inline int input_kind(const GemvJob &j) {
    return j.xf ? (j.xf2 ? IN_SWIGLU : j.norm_w ? IN_NORM : IN_F32) : IN_CODES;
}

}  // namespace
}  // namespace kh
