// GQA decode attention over a device-resident KV cache, split along the
// sequence: one launch computes per-split partial softmax sums, a second
// merges them.
//
// Reference: model::attend (crates/llm/src/model/mod.rs:769-819) with
// tensor::dot (tensor.rs:220-235) and softmax_inplace (tensor.rs:297-308).
// The reference walks every cached key once per query head; here a workgroup
// owns one KV head's query heads (up to 16 of them) and a run of P positions,
// and reads each key and value row once for the whole group -- the
// restructuring the reference's notes ask for (docs/engine.md:783-791).
//
// Split kernel, workgroup (split j, head group): all its K and V rows are
// loaded up front; scores s = dot(q, k) * scale; local max m_j,
// l_j = sum exp(s - m_j), acc_j = sum exp(s - m_j) v, the smallest score,
// and the scores themselves.  When one split covers the whole sequence it
// finishes the job itself with the reference's exact weights
// w = exp(s - M) * (1/S), dropping w < 1e-8 (mod.rs:807).
//
// Merge kernel, one workgroup per query head:
//   M = max m_j,  S = sum l_j exp(m_j - M),  acc = sum exp(m_j - M) acc_j,
// and out = acc * (1/S), less the terms the reference skips: splits whose
// largest weight is under 1e-8 are left out, and in the splits that straddle
// the threshold the stored scores name the skipped positions, whose
// w * v are taken back out (merge_head).
//
// The two launches share nothing but the partials in device memory, so no
// workgroup waits on another and no cross-XCD fence is needed.  Every sum has
// a fixed order, so results are deterministic run to run.
#include "common.hpp"

namespace kh {
namespace {

constexpr unsigned RSRC_WORD3 = 0x00020000;
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t rsrc(const void *p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)(bytes > 0xffffffffu ? 0xffffffffu : bytes), RSRC_WORD3);
}

struct AttnArgs {
    const float *q;
    const float *k;
    const float *v;
    size_t kstride, vstride;  // floats between consecutive positions
    int n_head, group, gc;    // group = n_head / n_kv_head; gc = heads per workgroup
    int L, P, nsplit;
    int nw;                   // waves per split workgroup: P = 16 R nw
    // when set, the length is read here (+ plus_one) and L/nsplit above are
    // the launch's maxima; splits past the length return at once
    const int32_t *len_dev;
    int plus_one;
    float scale;
    // per split, [nsplit][n_head]: local max, sum, smallest score; acc
    // [nsplit][n_head][hd]; scores [nsplit][n_head][P]
    float *pm, *pl, *pmin, *pacc, *psc;
    float *out;               // [n_head][hd]
    // batched rows (Transformer::forward_each, llama.rs:418-434): when set,
    // workgroup row z = blockIdx.z attends with rows[z] (its own cache and
    // length), its q and out rows z, and partials offset by z * row_floats
    const AttnRow *rows;
    size_t row_floats;
    // the session's step with RoPE and the cache push fused (when kraw is
    // set): q holds the new position's query unrotated; position L - 1's key
    // is RoPE(k_norm(kraw)) and its value vraw, both written into the caches
    // (kw, vw) at L - 1 by the split that holds it
    AttnRope rope;
    float *kw, *vw;
};

// The row of a batched launch: its cache, its length and its slices.
__device__ __forceinline__ void at_row(AttnArgs &a, int hd) {
    if (!a.rows) return;
    const int z = blockIdx.z;
    const AttnRow r = a.rows[z];
    a.k = r.k;
    a.v = r.v;
    a.L = r.L;
    a.q += (size_t)z * a.n_head * hd;
    a.out += (size_t)z * a.n_head * hd;
    const size_t o = (size_t)z * a.row_floats;
    a.pm += o, a.pl += o, a.pmin += o, a.pacc += o, a.psc += o;
    a.kw = r.k;
    a.vw = r.v;
    if (a.rope.kraw) {
        a.rope.kraw += (size_t)z * a.rope.raw_stride;
        a.rope.vraw += (size_t)z * a.rope.raw_stride;
    }
}

// Sums (or maxima) over the wave's four rows of 16 lanes, by swapping
// rows (v_permlane16_swap) and then halves (v_permlane32_swap) between two
// copies of a value; every lane gets the total, in a fixed order.  Written
// as inline assembly: the compiler folds the builtins' two results into one
// when both inputs are the same value.
__device__ __forceinline__ void swap16(float &a, float &b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(float &a, float &b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
template <typename F>
__device__ __forceinline__ float rows_reduce(float x, F op) {
    float a = x, b = x;
    swap16(a, b);
    x = op(a, b);
    a = x, b = x;
    swap32(a, b);
    return op(a, b);
}
__device__ __forceinline__ float rows_sum(float x) {
    return rows_reduce(x, [](float u, float v) { return u + v; });
}
__device__ __forceinline__ float rows_max(float x) {
    return rows_reduce(x, [](float u, float v) { return fmaxf(u, v); });
}
__device__ __forceinline__ float rows_min(float x) {
    return rows_reduce(x, [](float u, float v) { return fminf(u, v); });
}
// Split kernel, on matrix cores (v_mfma_f32_16x16x4_f32).  A workgroup of
// four waves owns one KV head's G <= 16 query heads and P = 64 R positions;
// wave w takes R tiles of 16 consecutive positions.  Per tile:
//   scores  S = K Q^T: A = 16 positions x 4 k-slots, B = 4 k-slots x 16
//           heads; in product m (of HD/16) k-slot c of lane (c, i) takes
//           the head dims 16m + 4c .. 16m + 4c + 3 (q dealt the same way),
//           so one load instruction reads 64 contiguous bytes of each of
//           the 16 key rows; the 16 columns are the G query heads (the rest
//           zero).
//   S lands as lane (c, j) holding positions 4c .. 4c+3 of head j: after
//   exp, exactly the A operand of the value product for the four position
//   groups r = 0..3 (position 4c + r in k-slot c).
//   values  O += P V: B = V rows 4c + r, lane (c, j) holding dims
//           4j .. 4j+3 (+64): one float4 of a row per lane, four rows of
//           256 contiguous bytes per load instruction.
// Every K and V row of the workgroup is loaded up front.  Statistics per
// head are reduced over the wave's four lane rows with lane swaps; the four
// waves meet once in LDS, as partial (m, l, acc) per split, or, when one
// split covers the whole sequence, as the reference's exact weights
// w = exp(s - M) * (1/S) with w < 1e-8 dropped (mod.rs:805-812).
typedef float f4v __attribute__((ext_vector_type(4)));

// One head held by a wave as dims lane + 64 e: rms_norm with `nw`
// (norm_heads, llama.rs:122-127; none when null), then RoPE at position pos
// (Rope::apply / apply_interleaved, tensor.rs:437-472), in place.
template <int HD>
struct RopeVals {
    static constexpr int HE = HD / 64;
    float w[HE], c[HE], sn[HE];  // norm weights (1 when none), cos and sin of the lane's dims
};
// The values norm_rope_head multiplies by: loaded apart from the arithmetic,
// so a kernel can issue these loads ahead of others it waits on first.
template <int HD>
__device__ __forceinline__ void rope_vals_load(RopeVals<HD> &v, const float *nw, const AttnRope &rp, int lane, int pos) {
    constexpr int HE = HD / 64;
    const int half = HD / 2;
#pragma unroll
    for (int e = 0; e < HE; e++) {
        const int d = lane + 64 * e;
        const int ip = rp.interleaved ? d >> 1 : d % half;
        v.w[e] = nw ? nw[d] : 1.0f;
        v.c[e] = rp.cos_t[(size_t)pos * half + ip];
        v.sn[e] = rp.sin_t[(size_t)pos * half + ip];
    }
}
template <int HD>
__device__ __forceinline__ void norm_rope_vals(float (&x)[HD / 64], const RopeVals<HD> &v, bool normed,
                                               const AttnRope &rp, int lane) {
    constexpr int HE = HD / 64;
    const int half = HD / 2;
    if (normed) {
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < HE; e++) {
            const float sq = x[e] * x[e];
            ss = ss + sq;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss = ss + __shfl_xor(ss, o);
        const float inv = 1.0f / sqrtf(ss / (float)HD + rp.eps);
#pragma unroll
        for (int e = 0; e < HE; e++) {
            const float u = x[e] * inv;
            x[e] = u * v.w[e];
        }
    }
    float out[HE];
#pragma unroll
    for (int e = 0; e < HE; e++) {
        const int d = lane + 64 * e;
        // the pair partner: dim d +- half (half split) or d ^ 1 (interleaved)
        float pv;
        if (rp.interleaved) {
            pv = __shfl_xor(x[e], 1);
        } else {
            if constexpr (HD == 128) pv = x[e ^ 1];  // d and d + 64 sit in one lane
            else pv = __shfl_xor(x[e], 32);
        }
        const bool first = rp.interleaved ? (d & 1) == 0 : d < half;
        const float c = v.c[e], sn = v.sn[e];
        if (first) {  // a = x, b = partner: a c - b s
            const float ac = x[e] * c, bs = pv * sn;
            out[e] = ac - bs;
        } else {      // b = x, a = partner: b c + a s
            const float bc = x[e] * c, as = pv * sn;
            out[e] = bc + as;
        }
    }
#pragma unroll
    for (int e = 0; e < HE; e++) x[e] = out[e];
}
template <int HD>
__device__ __forceinline__ void norm_rope_head(float (&x)[HD / 64], const float *nw, const AttnRope &rp, int lane,
                                               int pos) {
    RopeVals<HD> v;
    rope_vals_load<HD>(v, nw, rp, lane, pos);
    norm_rope_vals<HD>(x, v, nw != nullptr, rp, lane);
}

// Fused RoPE (the session's step).  Wave w takes heads w, w + NW, ...: the
// G query heads, then (in the workgroup holding the new position) the KV
// head's new key as head G; lane l holds dims l (+ 64) of the head, loaded
// with its norm weights, cos and sin (and the new value) ahead of the K and
// V loads, and rotated while they fly.
template <int HD, int NW>
struct RopeIn {
    static constexpr int RH = (16 + NW) / NW;  // heads per wave (at most G + 1 <= 17 heads)
    static constexpr int HE = HD / 64;         // dims per lane
    float x[RH][HE];
    RopeVals<HD> v[RH];                        // their norm weights, cos and sin
    float vnew;                                // the new value's dim tid (tid < HD, holding split)
};

template <int HD, int NW>
__device__ __forceinline__ void rope_load(const AttnArgs &a, RopeIn<HD, NW> &r, int wave, int lane, int G, int h0,
                                          int kvh, bool holds, int pos, int tid) {
#pragma unroll
    for (int i = 0; i < RopeIn<HD, NW>::RH; i++) {
        const int h = wave + i * NW;
#pragma unroll
        for (int e = 0; e < RopeIn<HD, NW>::HE; e++) r.x[i][e] = 0.0f;
        if (h < G || (h == G && holds)) {  // uniform per wave
            const float *src = h < G ? a.q + (size_t)(h0 + h) * HD : a.rope.kraw + (size_t)kvh * HD;
#pragma unroll
            for (int e = 0; e < RopeIn<HD, NW>::HE; e++) r.x[i][e] = src[lane + 64 * e];
            rope_vals_load<HD>(r.v[i], h < G ? a.rope.q_norm : a.rope.k_norm, a.rope, lane, pos);
        }
    }
    r.vnew = holds && tid < HD ? a.rope.vraw[(size_t)kvh * HD + tid] : 0.0f;
}

// Per head: norm_rope_head into s_rot[head]; when `holds`, the new key
// (s_rot[G]) and value (s_vnew) are also written into the caches at pos.
// The caller syncs the workgroup before reading s_rot / s_vnew.
template <int HD, int NW>
__device__ __forceinline__ void rope_apply(const AttnArgs &a, const RopeIn<HD, NW> &r, float (*s_rot)[HD],
                                           float *s_vnew, int wave, int lane, int tid, int G, int kvh, int pos,
                                           bool holds) {
    constexpr int HE = RopeIn<HD, NW>::HE;
#pragma unroll
    for (int i = 0; i < RopeIn<HD, NW>::RH; i++) {
        const int h = wave + i * NW;
        if (!(h < G || (h == G && holds))) continue;  // uniform per wave
        float x[HE];
#pragma unroll
        for (int e = 0; e < HE; e++) x[e] = r.x[i][e];
        norm_rope_vals<HD>(x, r.v[i], (h < G ? a.rope.q_norm : a.rope.k_norm) != nullptr, a.rope, lane);
#pragma unroll
        for (int e = 0; e < HE; e++) {
            const int d = lane + 64 * e;
            s_rot[h][d] = x[e];
            if (h == G) a.kw[(size_t)pos * a.kstride + (size_t)kvh * HD + d] = x[e];
        }
    }
    if (holds && tid < HD) {  // NW >= 2 waves: one dim a thread
        s_vnew[tid] = r.vnew;
        a.vw[(size_t)pos * a.vstride + (size_t)kvh * HD + tid] = r.vnew;
    }
}

// Rows::Following (a prompt read a pass at a time, run_rows with
// llama.rs:249-257): every row's query and key heads normed and rotated at
// the row's own position, each row's key and value pushed into the cache
// row at that position.  The attention launch that follows reads the
// rotated queries in q and the cache; no row's attention may start before
// every row of the pass is pushed, which is why this is a launch of its own
// and not fused into the split kernel as in the one-token step.
// Grid (n_head + n_kv_head, rows): one wave per head of a row; row i is at
// position rows[i].L - 1 of cache (rows[i].k, rows[i].v).
template <int HD>
__global__ __launch_bounds__(64) void rope_push_rows_kernel(float *q, const float *k, const float *v,
                                                            const AttnRow *rows, AttnRope rp, int n_head,
                                                            int n_kv_head, size_t kstride, size_t vstride) {
    constexpr int HE = HD / 64;
    const int h = blockIdx.x, i = blockIdx.y, lane = threadIdx.x;
    const AttnRow r = rows[i];
    const int pos = r.L - 1;
    float x[HE];
    if (h < n_head) {
        float *src = q + ((size_t)i * n_head + h) * HD;
#pragma unroll
        for (int e = 0; e < HE; e++) x[e] = src[lane + 64 * e];
        norm_rope_head<HD>(x, rp.q_norm, rp, lane, pos);
#pragma unroll
        for (int e = 0; e < HE; e++) src[lane + 64 * e] = x[e];
        return;
    }
    const int kvh = h - n_head;
    const float *ks = k + ((size_t)i * n_kv_head + kvh) * HD;
    const float *vs = v + ((size_t)i * n_kv_head + kvh) * HD;
#pragma unroll
    for (int e = 0; e < HE; e++) x[e] = ks[lane + 64 * e];
    norm_rope_head<HD>(x, rp.k_norm, rp, lane, pos);
    float *kd = r.k + (size_t)pos * kstride + (size_t)kvh * HD;
    float *vd = r.v + (size_t)pos * vstride + (size_t)kvh * HD;
#pragma unroll
    for (int e = 0; e < HE; e++) {
        kd[lane + 64 * e] = x[e];
        vd[lane + 64 * e] = vs[lane + 64 * e];
    }
}


// The fields the first loads need lead the arguments, which are preloaded
// into scalar registers (the build's kernarg preload): the device length's
// load is issued at once, and the key, value and query loads wait on no
// scalar load.  ROWS (batched rows, or fields too wide for the words) takes
// them from the argument struct and the row table instead.  gg: group | gc
// << 15 | plus_one << 31.
template <int HD, int R, int NW, bool ROPE, bool ROWS>
__global__ __launch_bounds__(64 * NW) void attn_split_kernel(const int32_t *len_dev, const float *k0, const float *v0,
                                                             const float *q0, unsigned kst0, unsigned vst0, int L0,
                                                             unsigned gg, AttnArgs a) {
    const int len_raw = len_dev ? *len_dev : 0;
    if constexpr (ROWS) {
        at_row(a, HD);
    } else {
        a.k = k0, a.v = v0, a.q = q0, a.kstride = kst0, a.vstride = vst0, a.L = L0;
        a.group = (int)(gg & 0x7fffu), a.gc = (int)((gg >> 15) & 0x7fffu), a.plus_one = (int)(gg >> 31);
    }
    constexpr int NQ4 = HD / 16;  // float4s per lane of a key row: products of 16 dims
    constexpr int VT = HD / 64;  // float4s per lane of a value row
    constexpr int NT = HD / 16;  // 16-column tiles of the output
    constexpr int P = 16 * R * NW;
    constexpr int NTH = 64 * NW;
    const int split = blockIdx.x, hg = blockIdx.y;
    const int G = a.gc;
    const int h0 = hg * G, kvh = h0 / a.group;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j16 = lane & 15, c4 = lane >> 4;
    const int L = len_dev ? min(len_raw + a.plus_one, a.L) : a.L;
    const int nsplit = (L + P - 1) / P;
    if (split >= nsplit) return;
    const int t0 = split * P;
    const int n = min(L - t0, P);
    const bool whole = nsplit == 1;
    const rsrc_t K = rsrc(a.k, (size_t)L * a.kstride * 4), V = rsrc(a.v, (size_t)L * a.vstride * 4);
    const int pw = wave * 16 * R;  // the wave's first position in the split

    __shared__ __align__(16) float s_acc[NW][16][HD];  // per-wave totals
    __shared__ float s_st[3][NW][16];                  // per-wave max, sum, smallest score
    // over the waves in wave order: the largest of row st, the total of row st
    auto wmax = [&](int st, int h) {
        float x = s_st[st][0][h];
#pragma unroll
        for (int w = 1; w < NW; w++) x = fmaxf(x, s_st[st][w][h]);
        return x;
    };
    auto wmin = [&](int st, int h) {
        float x = s_st[st][0][h];
#pragma unroll
        for (int w = 1; w < NW; w++) x = fminf(x, s_st[st][w][h]);
        return x;
    };

    // q first (the score products wait on it before any key), then keys,
    // then values: loads complete in issue order
    const bool hv = j16 < G;
    f4v qb4[NQ4];
    // fused RoPE: the query heads (and, in the split holding the new
    // position, the new key) loaded now, rotated once K and V are in flight
    constexpr bool rope = ROPE;  // launched with the rope argument set
    const int pos = L - 1;
    const bool holds = rope && pos >= t0 && pos < t0 + P;
    RopeIn<HD, NW> xr;
    if (rope) {
        rope_load<HD, NW>(a, xr, wave, lane, G, h0, kvh, holds, pos, tid);
    } else {
        const float *qh = a.q + (size_t)(h0 + (hv ? j16 : 0)) * HD + 4 * c4;
#pragma unroll
        for (int m = 0; m < NQ4; m++) {
            const float4 f = *reinterpret_cast<const float4 *>(qh + 16 * m);
            qb4[m] = hv ? f4v{f.x, f.y, f.z, f.w} : f4v{0.f, 0.f, 0.f, 0.f};
        }
    }
    f4v kq[R][NQ4];
    f4v vv[R][4][VT];
#pragma unroll
    for (int u = 0; u < R; u++) {
        const size_t t = (size_t)(t0 + pw + 16 * u + j16);
        const unsigned off = (unsigned)((t * a.kstride + (size_t)kvh * HD + 4 * c4) * 4);
#pragma unroll
        for (int m = 0; m < NQ4; m++)
            kq[u][m] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(K, off, 64 * m, 0));
    }
#pragma unroll
    for (int u = 0; u < R; u++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const size_t t = (size_t)(t0 + pw + 16 * u + 4 * c4 + r);
            const unsigned off = (unsigned)((t * a.vstride + (size_t)kvh * HD + 4 * j16) * 4);
#pragma unroll
            for (int v = 0; v < VT; v++)
                vv[u][r][v] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(V, off, 256 * v, 0));
        }
    // every key and value load is issued before any score is computed: left
    // to itself the scheduler interleaves them with the products and drains
    // the queue between batches, a round trip each
    __builtin_amdgcn_sched_barrier(0);

    if (rope) {
        __shared__ __align__(16) float s_rot[17][HD];
        __shared__ __align__(16) float s_vnew[HD];
        rope_apply<HD, NW>(a, xr, s_rot, s_vnew, wave, lane, tid, G, kvh, pos, holds);
        __syncthreads();
        const float *qh = &s_rot[hv ? j16 : 0][4 * c4];
#pragma unroll
        for (int m = 0; m < NQ4; m++) {
            const float4 f = *reinterpret_cast<const float4 *>(qh + 16 * m);
            qb4[m] = hv ? f4v{f.x, f.y, f.z, f.w} : f4v{0.f, 0.f, 0.f, 0.f};
        }
        if (holds) {  // the new position's key and value, in place of the cache's old row
#pragma unroll
            for (int u = 0; u < R; u++) {
                const bool mine = t0 + pw + 16 * u + j16 == pos;
#pragma unroll
                for (int m = 0; m < NQ4; m++) {
                    const float4 f = *reinterpret_cast<const float4 *>(&s_rot[G][16 * m + 4 * c4]);
                    if (mine) kq[u][m] = f4v{f.x, f.y, f.z, f.w};
                }
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const bool vmine = t0 + pw + 16 * u + 4 * c4 + r == pos;
#pragma unroll
                    for (int v = 0; v < VT; v++) {
                        const float4 f = *reinterpret_cast<const float4 *>(&s_vnew[64 * v + 4 * j16]);
                        if (vmine) vv[u][r][v] = f4v{f.x, f.y, f.z, f.w};
                    }
                }
            }
        }
    }

    // scores: lane (c4, j16) holds positions pw + 16u + 4c4 + r of head j16
    f4v s[R];
    float mx = -INFINITY, mn = INFINITY;
#pragma unroll
    for (int u = 0; u < R; u++) {
        f4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < NQ4; m++)
#pragma unroll
            for (int c = 0; c < 4; c++) d = __builtin_amdgcn_mfma_f32_16x16x4f32(kq[u][m][c], qb4[m][c], d, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const bool ok = hv && pw + 16 * u + 4 * c4 + r < n;
            const float sc = d[r] * a.scale;  // dot(q, k) * scale, mod.rs:802
            s[u][r] = ok ? sc : -INFINITY;
            mx = fmaxf(mx, s[u][r]);
            mn = ok ? fminf(mn, sc) : mn;
        }
    }
    mx = rows_max(mx);
    mn = rows_min(mn);

    // O = sum_t p_t v_t over the wave's tiles, p given in the score layout
    auto values = [&](const f4v (&p)[R], f4v (&acc)[NT]) {
#pragma unroll
        for (int q = 0; q < NT; q++) acc[q] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < R; u++)
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int q = 0; q < NT; q++)
                    acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[u][r], vv[u][r][q >> 2][q & 3], acc[q], 0, 0, 0);
    };
    // acc[q][i] is head 4 c4 + i, dim 4 j16 + (q & 3) + 64 (q >> 2)
    auto store_acc = [&](const f4v (&acc)[NT]) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int h = 4 * c4 + i;
            if (h < G) {
#pragma unroll
                for (int v = 0; v < VT; v++)
                    *reinterpret_cast<float4 *>(&s_acc[wave][h][64 * v + 4 * j16]) =
                        make_float4(acc[4 * v][i], acc[4 * v + 1][i], acc[4 * v + 2][i], acc[4 * v + 3][i]);
            }
        }
    };

    // exp(s - m) against the wave's max
    f4v e[R];
    float l = 0.0f;
#pragma unroll
    for (int u = 0; u < R; u++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            e[u][r] = s[u][r] == -INFINITY ? 0.0f : expf(s[u][r] - mx);
            l += e[u][r];
        }
    l = rows_sum(l);
    if (!whole) {
        f4v acc[NT];
        values(e, acc);
        store_acc(acc);
        if (c4 == 0 && hv) {
            s_st[0][wave][j16] = mx;
            s_st[1][wave][j16] = l;
            s_st[2][wave][j16] = mn;
        }
        __syncthreads();
        // the split's statistics: M over the waves, each wave rescaled to it
        for (int i = tid; i < G * HD; i += NTH) {
            const int h = i / HD, d = i % HD;
            const float M = wmax(0, h);
            float x = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float c = s_st[0][w][h] == -INFINITY ? 0.0f : expf(s_st[0][w][h] - M);
                x = fmaf(c, s_acc[w][h][d], x);
            }
            a.pacc[((size_t)split * a.n_head + h0 + h) * HD + d] = x;
        }
        if (tid < G) {
            const int h = tid;
            const float M = wmax(0, h);
            float Ls = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float c = s_st[0][w][h] == -INFINITY ? 0.0f : expf(s_st[0][w][h] - M);
                Ls = fmaf(c, s_st[1][w][h], Ls);
            }
            const size_t o = (size_t)split * a.n_head + h0 + h;
            a.pm[o] = M;
            a.pl[o] = Ls;
            a.pmin[o] = wmin(2, h);
        }
        // the scores, for the merge's decision on the reference's 1e-8 skip
        // (stored last: a store ahead of a load would hold up its wait)
        if (hv) {
            float *ps = a.psc + ((size_t)split * a.n_head + h0 + j16) * P + pw + 4 * c4;
#pragma unroll
            for (int u = 0; u < R; u++)
                *reinterpret_cast<float4 *>(ps + 16 * u) = make_float4(s[u][0], s[u][1], s[u][2], s[u][3]);
        }
        return;
    }

    // One split is the whole sequence: the reference's own weights
    // w = exp(s - M) * (1/S), S = sum exp(s - M), dropping w < 1e-8
    // (softmax_inplace, tensor.rs:297-308; mod.rs:805-812).
    if (c4 == 0 && hv) s_st[0][wave][j16] = mx;
    __syncthreads();
    const int hj = hv ? j16 : 0;
    const float M = wmax(0, hj);
    l = 0.0f;
#pragma unroll
    for (int u = 0; u < R; u++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            e[u][r] = s[u][r] == -INFINITY ? 0.0f : expf(s[u][r] - M);
            l += e[u][r];
        }
    l = rows_sum(l);
    if (c4 == 0 && hv) s_st[1][wave][j16] = l;
    __syncthreads();
    float S = s_st[1][0][hj];
#pragma unroll
    for (int w = 1; w < NW; w++) S = S + s_st[1][w][hj];
    const float inv = 1.0f / S;
#pragma unroll
    for (int u = 0; u < R; u++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float w = e[u][r] * inv;
            e[u][r] = w < 1e-8f ? 0.0f : w;
        }
    f4v acc[NT];
    values(e, acc);
    store_acc(acc);
    __syncthreads();
    for (int i = tid; i < G * HD; i += NTH) {
        const int h = i / HD, d = i % HD;
        float x = s_acc[0][h][d];
#pragma unroll
        for (int w = 1; w < NW; w++) x = x + s_acc[w][h][d];
        a.out[(size_t)(h0 + h) * HD + d] = x;
    }
}

// Fixed-order butterfly within each wave, then the four wave results in wave
// order; every thread gets the result.  s_w holds four floats.
template <typename F>
__device__ __forceinline__ float block_reduce(float v, float *s_w, F op) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o));
    if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = v;
    __syncthreads();
    return op(op(s_w[0], s_w[1]), op(s_w[2], s_w[3]));
}

constexpr int MAX_SPLITS = 4096;

// Exclusive prefix sum of one int per thread over the workgroup (256
// threads); *total gets the sum.  s holds four ints and is free again on return.
__device__ __forceinline__ int block_excl_scan(int v, int *s, int *total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    if (lane == 63) s[wv] = x;
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const int t = s[w];
        off += w < wv ? t : 0;
        tot += t;
    }
    *total = tot;
    __syncthreads();
    return off + x - v;
}

// The merge of one head's splits (one workgroup of 256 threads), over the
// head's dims [d0, d0 + D):
//   M = max m_j,  S = sum_j l_j e^{m_j - M},  out = sum_j e^{m_j - M} acc_j / S,
// less the terms the reference skips, w_t = e^{s_t - M} * (1/S) < 1e-8
// (mod.rs:807).  Decided per split from its extremes: a split whose largest
// weight is under 1e-8 is left out whole; one whose smallest is not is taken
// whole; the straddling ones have their stored scores read, 1024 candidates
// at a time, and the value rows of just the skipped positions are gathered,
// all loads in flight together, and taken back out.  The first splits'
// partial values are loaded before M is known, so their latency overlaps the
// reductions.  vrow(t, q) is float4 q of position t's value row for this
// head.  Every list is compacted in index order and every sum has a fixed
// order.
template <int HD, int D, typename VRow>
__device__ __forceinline__ void merge_head(const float *pm, const float *pl, const float *pmin, const float *pacc,
                                           const float *psc, int ns, int n_head, int h, int d0, int P, int L,
                                           VRow vrow, float *out) {
    constexpr int NQ = D / 4, NSG = 256 / NQ;  // float4 slices of the dims; split (or position) groups
    constexpr int PER = MAX_SPLITS / 256;      // splits per thread at most
    constexpr int CAP = 2048;                  // skipped positions gathered per flush
    constexpr int NB = 8;                      // partial values in flight per thread
    const int tid = threadIdx.x;
    __shared__ float s_w[2][4];
    __shared__ int s_scan[4];
    __shared__ float s_c[MAX_SPLITS];           // e^{m_j - M}, or 0 for a split left out
    __shared__ int s_list[MAX_SPLITS];          // straddling splits, in index order
    __shared__ __align__(16) float s_acc[NSG][D];
    __shared__ __align__(16) float s_fix[NSG][D];
    __shared__ int s_kpos[CAP];
    __shared__ float s_kw[CAP];

    const int sg = tid / NQ, dq = tid % NQ;
    // each thread a run of splits, its statistics held in registers: loaded
    // first (the reductions below wait on them, and loads complete in issue
    // order), as buffer loads that read zero past the last split, under a
    // bound uniform over the workgroup, so no load waits on a branch
    const int per = (ns + 255) / 256, i0 = tid * per, n = min(ns - i0, per);
    const size_t sbytes = (size_t)ns * n_head * 4;
    const rsrc_t PM = rsrc(pm, sbytes), PL = rsrc(pl, sbytes), PN = rsrc(pmin, sbytes);
    float m[PER], l[PER], mn[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        if (u < per) {
            const unsigned o = (unsigned)(((size_t)(i0 + u) * n_head + h) * 4);
            m[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(PM, o, 0, 0));
            l[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(PL, o, 0, 0));
            mn[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(PN, o, 0, 0));
        }
    }
    const rsrc_t PA = rsrc(pacc, (size_t)ns * n_head * HD * 4);
    auto pa_load = [&](int i) {  // zeros past the last split (buffer range)
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                              PA, (unsigned)((((size_t)i * n_head + h) * HD + d0 + 4 * dq) * 4), 0, 0));
    };
    float4 v[NB];
#pragma unroll
    for (int u = 0; u < NB; u++) v[u] = pa_load(sg + u * NSG);

    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < PER; u++)
        if (u < n) mx = fmaxf(mx, m[u]);
    const float M = block_reduce(mx, s_w[0], [](float x, float y) { return fmaxf(x, y); });
    float s = 0.0f;
    float c[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        if (u < n) {
            c[u] = expf(m[u] - M);
            s = fmaf(l[u], c[u], s);
        }
    }
    const float S = block_reduce(s, s_w[1], [](float x, float y) { return x + y; });
    const float inv = 1.0f / S;  // inv = 1 / sum, tensor.rs:304

    unsigned mask = 0;  // straddling splits of this thread's run
#pragma unroll
    for (int u = 0; u < PER; u++) {
        if (u < n) {
            const bool out_whole = c[u] * inv < 1e-8f;  // every weight of the split is skipped
            s_c[i0 + u] = out_whole ? 0.0f : c[u];
            if (!out_whole && expf(mn[u] - M) * inv < 1e-8f) mask |= 1u << u;
        }
    }
    int nstr;
    int at = block_excl_scan(__builtin_popcount(mask), s_scan, &nstr);  // its barrier publishes s_c
    if (nstr) {
#pragma unroll
        for (int u = 0; u < PER; u++)
            if (mask >> u & 1u) s_list[at++] = i0 + u;
    }

    // acc[d] = sum_j c_j acc_j[d]: thread (split group sg, float4 slice dq)
    // walks splits sg, sg + NSG, ..., NB loads at a time
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j0 = sg;; ) {
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const int i = j0 + u * NSG;
            const float cu = i < ns ? s_c[i] : 0.0f;
            x.x = fmaf(cu, v[u].x, x.x);
            x.y = fmaf(cu, v[u].y, x.y);
            x.z = fmaf(cu, v[u].z, x.z);
            x.w = fmaf(cu, v[u].w, x.w);
        }
        j0 += NB * NSG;
        if (j0 >= ns) break;
#pragma unroll
        for (int u = 0; u < NB; u++) v[u] = pa_load(j0 + u * NSG);
    }
    *reinterpret_cast<float4 *>(&s_acc[sg][4 * dq]) = x;

    // the skipped terms of the straddling splits: 1024 candidates a batch,
    // four consecutive positions of one split per thread
    float4 fix = make_float4(0.f, 0.f, 0.f, 0.f);
    if (nstr) {
        __syncthreads();  // s_list
        int nk = 0;       // listed skipped positions (the same in every thread)
        const int ncand = nstr * P;
        for (int c0 = 0; c0 < ncand; c0 += 1024) {
            const int cand = c0 + 4 * tid;
            float w4[4] = {0.f, 0.f, 0.f, 0.f};
            int t0 = 0, cnt = 0;
            if (cand < ncand) {
                const int j = s_list[cand / P], k = cand % P;
                t0 = j * P + k;
                const float4 sc4 = *reinterpret_cast<const float4 *>(psc + ((size_t)j * n_head + h) * P + k);
                const float sc[4] = {sc4.x, sc4.y, sc4.z, sc4.w};
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    if (t0 + u < L && sc[u] != -INFINITY) {
                        float w = expf(sc[u] - M);
                        w = w * inv;
                        // kept (a weight that underflows to 0 adds nothing either)
                        w4[u] = w < 1e-8f ? w : 0.0f;
                        cnt += w4[u] > 0.0f;
                    }
                }
            }
            int added;
            int o = nk + block_excl_scan(cnt, s_scan, &added);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (w4[u] > 0.0f) {
                    s_kpos[o] = t0 + u;
                    s_kw[o] = w4[u];
                    o++;
                }
            }
            nk += added;
            __syncthreads();
            if (nk > CAP - 1024 || c0 + 1024 >= ncand) {
                // gather: thread (group sg, slice dq) takes listed positions sg, sg + NSG, ...
                for (int k0 = sg; k0 < nk; k0 += 4 * NSG) {
                    float4 vv[4];
                    float ww[4];
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int kk = k0 + u * NSG;
                        const bool ok = kk < nk;
                        vv[u] = vrow(s_kpos[ok ? kk : 0], d0 / 4 + dq);
                        ww[u] = ok ? s_kw[kk] : 0.0f;
                    }
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        fix.x = fmaf(ww[u], vv[u].x, fix.x);
                        fix.y = fmaf(ww[u], vv[u].y, fix.y);
                        fix.z = fmaf(ww[u], vv[u].z, fix.z);
                        fix.w = fmaf(ww[u], vv[u].w, fix.w);
                    }
                }
                nk = 0;
                __syncthreads();
            }
        }
        *reinterpret_cast<float4 *>(&s_fix[sg][4 * dq]) = fix;
    }
    __syncthreads();
    if (tid < NQ) {
        float4 x = *reinterpret_cast<const float4 *>(&s_acc[0][4 * tid]);
#pragma unroll
        for (int g = 1; g < NSG; g++) {
            const float4 y = *reinterpret_cast<const float4 *>(&s_acc[g][4 * tid]);
            x = make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
        }
        x = make_float4(x.x * inv, x.y * inv, x.z * inv, x.w * inv);
        if (nstr) {
            float4 f = *reinterpret_cast<const float4 *>(&s_fix[0][4 * tid]);
#pragma unroll
            for (int g = 1; g < NSG; g++) {
                const float4 z = *reinterpret_cast<const float4 *>(&s_fix[g][4 * tid]);
                f = make_float4(f.x + z.x, f.y + z.y, f.z + z.z, f.w + z.w);
            }
            x = make_float4(x.x - f.x, x.y - f.y, x.z - f.z, x.w - f.w);
        }
        *reinterpret_cast<float4 *>(out + (size_t)h * HD + d0 + 4 * tid) = x;
    }
}

// The partials' pointers, the length and the split size lead the arguments
// (preloaded, as the split kernel's): ROWS (batched rows, or head counts
// past 16 bits) takes them from the struct and the row table.  pn: P |
// plus_one << 31; hg: n_head | group << 16.
// The merge of dims d0 .. d0 + D of one head (rows of HD) without barriers,
// for up to merge_fast_max(D) splits (128 for 64 or 128 dims): every
// load is issued at once (each wave reads every split's max, sum and
// minimum, four splits a lane, and its quarter of the dims of every split's
// partial values, D / 16 float4s a lane-row of 64 / (D / 16) splits), the maximum and the sum are
// wave butterflies (each wave computes the same ones, in the same order),
// the weights e^{m_j - M} pass through the wave's own LDS row, and the
// split groups' sums meet by butterfly.  Returns false, having written
// nothing, when a split straddles the 1e-8 line (some but not all of its
// weights skipped): the caller then runs merge_head, which handles those.
// The most splits merge_head_fast takes for D dims: its partial values'
// split groups and its statistics' four splits a lane both cover them, and
// no more than 128: the more splits, the likelier one straddles the 1e-8
// line, and a straddle costs the fast path's loads on top of merge_head's
// (latent attention at L = 32768, 256 splits of random data: 40.8 -> 43.2 us
// per layer when taken).
constexpr int merge_fast_max(int d) { return 16 * 64 / (d / 16) < 128 ? 16 * 64 / (d / 16) : 128; }
template <int HD, int D>
__device__ __forceinline__ bool merge_head_fast(const float *pm, const float *pl, const float *pmin, const float *pacc,
                                                int ns, int n_head, int h, int d0, float *out) {
    constexpr int NQ = D / 16;      // float4s of a wave's dims
    constexpr int SG = 64 / NQ;     // split groups a wave-row holds
    constexpr int PJ = 16;          // partial values a lane holds at most
    constexpr int PS = 4;           // splits of statistics a lane holds
    __shared__ float s_c[4][PS * 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int dq = lane % NQ, sg = lane / NQ;
    const size_t sb = (size_t)ns * n_head * 4;
    const rsrc_t PM = rsrc(pm, sb), PL = rsrc(pl, sb), PN = rsrc(pmin, sb);
    const rsrc_t PA = rsrc(pacc, sb * HD);
    float m[PS], l[PS], mn[PS];
#pragma unroll
    for (int u = 0; u < PS; u++) {  // past the last split: out of range, zero
        const unsigned o = (unsigned)((((size_t)(lane + 64 * u)) * n_head + h) * 4);
        m[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(PM, o, 0, 0));
        l[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(PL, o, 0, 0));
        mn[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(PN, o, 0, 0));
    }
    float4 v[PJ];
    const int d = d0 + (D / 4) * wave + 4 * dq;
#pragma unroll
    for (int k = 0; k < PJ; k++) {  // split sg + SG k
        const unsigned o = (unsigned)((((size_t)(sg + SG * k) * n_head + h) * HD + d) * 4);
        v[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(PA, o, 0, 0));
    }
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < PS; u++)
        if (lane + 64 * u < ns) mx = fmaxf(mx, m[u]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float c[PS], sum = 0.0f;
#pragma unroll
    for (int u = 0; u < PS; u++) {
        c[u] = lane + 64 * u < ns ? expf(m[u] - mx) : 0.0f;
        sum = fmaf(l[u], c[u], sum);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum = sum + __shfl_xor(sum, o);
    const float inv = 1.0f / sum;  // inv = 1 / sum, tensor.rs:304
    bool straddle = false;
#pragma unroll
    for (int u = 0; u < PS; u++) {
        if (lane + 64 * u < ns) {
            const bool out_whole = c[u] * inv < 1e-8f;  // every weight of the split is skipped
            if (!out_whole && expf(mn[u] - mx) * inv < 1e-8f) straddle = true;
            s_c[wave][lane + 64 * u] = out_whole ? 0.0f : c[u];
        }
    }
    if (__builtin_amdgcn_ballot_w64(straddle)) return false;  // the same in every wave
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");    // the wave's own LDS row
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < PJ; k++) {
        const int j = sg + SG * k;
        const float cj = j < ns ? s_c[wave][j] : 0.0f;
        x.x = fmaf(cj, v[k].x, x.x);
        x.y = fmaf(cj, v[k].y, x.y);
        x.z = fmaf(cj, v[k].z, x.z);
        x.w = fmaf(cj, v[k].w, x.w);
    }
#pragma unroll
    for (int o = NQ; o < 64; o <<= 1) {  // the split groups, lane bits above dq
        x.x = x.x + __shfl_xor(x.x, o);
        x.y = x.y + __shfl_xor(x.y, o);
        x.z = x.z + __shfl_xor(x.z, o);
        x.w = x.w + __shfl_xor(x.w, o);
    }
    if (sg == 0)
        *reinterpret_cast<float4 *>(out + (size_t)h * HD + d) = make_float4(x.x * inv, x.y * inv, x.z * inv, x.w * inv);
    return true;
}

template <int HD, bool ROWS>
__global__ __launch_bounds__(256) void attn_merge_kernel(const int32_t *len_dev, float *pm0, float *pl0, float *pmin0,
                                                         float *pacc0, int L0, unsigned pn, unsigned hg,
                                                         AttnArgs a) {
    const int len_raw = len_dev ? *len_dev : 0;
    if constexpr (ROWS) {
        at_row(a, HD);
    } else {
        a.n_head = (int)(hg & 0xffffu), a.group = (int)(hg >> 16);
        a.pm = pm0, a.pl = pl0, a.pmin = pmin0, a.pacc = pacc0, a.L = L0, a.P = (int)(pn & 0x7fffffffu), a.plus_one = (int)(pn >> 31);
    }
    const int h = blockIdx.x;
    const int L = len_dev ? min(len_raw + a.plus_one, a.L) : a.L;
    const int ns = (L + a.P - 1) / a.P;
    if (ns <= 1) return;  // the split kernel finished a single split itself
    const rsrc_t V = rsrc(a.v, (size_t)L * a.vstride * 4);
    const size_t voff = (size_t)(h / a.group) * HD;
    auto vrow = [&](int t, int d4) {
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                              V, (unsigned)(((size_t)t * a.vstride + voff + 4 * d4) * 4), 0, 0));
    };
    if (ns <= merge_fast_max(HD) && merge_head_fast<HD, HD>(a.pm, a.pl, a.pmin, a.pacc, ns, a.n_head, h, 0, a.out))
        return;
    merge_head<HD, HD>(a.pm, a.pl, a.pmin, a.pacc, a.psc, ns, a.n_head, h, 0, a.P, L, vrow, a.out);
}

// A prompt's pass (Rows::Following, run_rows llama.rs:258-271): n rows at
// consecutive positions of one cache, row i attending over positions
// 0 .. rows[i].L - 1, the rows already rotated and pushed.  A workgroup
// takes a tile of 16 columns -- 16 / gc rows x the gc query heads of a head
// group -- and its NW waves stream the keys and values once for all of
// them, wave w taking the 16-position tiles w, w + NW, ..., on the matrix
// cores in the split kernel's layouts (v_mfma_f32_16x16x4f32: S = K Q^T
// lands as lane (c, j) holding positions 4c .. 4c + 3 of column j; O += P V
// with V rows 4c + r).  Two passes over the positions: the column's maximum
// M and sum S = sum e^{s - M} (per wave a running maximum with the sum
// rescaled when it rises; the waves' (M, S) combined in LDS in wave order),
// then the reference's weights w = e^{s - M} * (1/S), w < 1e-8 dropped
// (mod.rs:805-812), times the values, the waves' sums added in LDS in wave
// order.  Every column's whole sequence is in one workgroup: no partials in
// memory and no merge launch.  Scores are dot(q, k) * scale (mod.rs:802).
struct PassArgs {
    const float *q;        // [n][n_head][HD]
    const AttnRow *rows;   // [n]: the cache (the same for every row) and each row's length
    float *out;            // [n][n_head][HD]
    size_t kstride, vstride;
    int n, n_head, group, gc;
    float scale;
};

template <int HD, int NW>
__global__ __launch_bounds__(64 * NW) void attn_pass_kernel(PassArgs a) {
    constexpr int NQ4 = HD / 16, VT = HD / 64, NT = HD / 16;
    constexpr int STEP = 16 * NW;  // positions between one wave's tiles
    const int tid = threadIdx.x, lane = tid & 63, j16 = lane & 15, c4 = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gc = a.gc, rpt = 16 / gc;
    const int r0 = blockIdx.x * rpt, h0 = blockIdx.y * gc, kvh = h0 / a.group;
    const int rlast = min(r0 + rpt, a.n) - 1;
    const AttnRow first = a.rows[0];
    const int L = a.rows[rlast].L;  // the longest sequence of the tile
    const rsrc_t K = rsrc(first.k, (size_t)L * a.kstride * 4), V = rsrc(first.v, (size_t)L * a.vstride * 4);
    // the lane's column: row r0 + j16 / gc, head h0 + j16 % gc
    const int cr = r0 + j16 / gc, ch = h0 + j16 % gc;
    const bool hv = j16 < rpt * gc && cr < a.n;
    const int last = hv ? a.rows[cr].L - 1 : -1;  // the column attends t <= last
    f4v qb4[NQ4];
    {
        const float *qh = a.q + ((size_t)(hv ? cr : r0) * a.n_head + (hv ? ch : h0)) * HD + 4 * c4;
#pragma unroll
        for (int m = 0; m < NQ4; m++) {
            const float4 f = *reinterpret_cast<const float4 *>(qh + 16 * m);
            qb4[m] = hv ? f4v{f.x, f.y, f.z, f.w} : f4v{0.f, 0.f, 0.f, 0.f};
        }
    }
    auto load_k = [&](int t0, f4v (&kq)[NQ4]) {
        const unsigned off = (unsigned)(((size_t)(t0 + j16) * a.kstride + (size_t)kvh * HD + 4 * c4) * 4);
#pragma unroll
        for (int m = 0; m < NQ4; m++)
            kq[m] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(K, off, 64 * m, 0));
    };
    auto load_v = [&](int t0, f4v (&vv)[4][VT]) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const unsigned off =
                (unsigned)(((size_t)(t0 + 4 * c4 + r) * a.vstride + (size_t)kvh * HD + 4 * j16) * 4);
#pragma unroll
            for (int v = 0; v < VT; v++)
                vv[r][v] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(V, off, 256 * v, 0));
        }
    };
    // scores of positions t0 + 4 c4 + r of the lane's column, -inf where masked
    auto scores = [&](int t0, const f4v (&kq)[NQ4], float (&s)[4]) {
        f4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < NQ4; m++)
#pragma unroll
            for (int c = 0; c < 4; c++) d = __builtin_amdgcn_mfma_f32_16x16x4f32(kq[m][c], qb4[m][c], d, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float sc = d[r] * a.scale;
            s[r] = t0 + 4 * c4 + r <= last ? sc : -INFINITY;
        }
    };
    // Both passes keep the wave's next tile in flight while one is worked
    // (tiles past L read zeros: the buffers' range ends at L).
    // pass 1: the maximum M and the sum of e^{s - M}
    float M = -INFINITY, S = 0.0f;
    auto stats = [&](int t0, const f4v (&kq)[NQ4]) {
        float s[4];
        scores(t0, kq, s);
        const float mx = rows_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
        const float Mn = fmaxf(M, mx);
        float e = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; r++) e += s[r] == -INFINITY ? 0.0f : expf(s[r] - Mn);
        e = rows_sum(e);
        S = (M == -INFINITY ? 0.0f : S * expf(M - Mn)) + e;
        M = Mn;
    };
    {
        f4v ka[NQ4], kb[NQ4];
        load_k(16 * wave, ka);
        for (int t0 = 16 * wave; t0 < L; t0 += 2 * STEP) {
            load_k(t0 + STEP, kb);
            stats(t0, ka);
            if (t0 + STEP >= L) break;
            load_k(t0 + 2 * STEP, ka);
            stats(t0 + STEP, kb);
        }
    }
    if constexpr (NW > 1) {  // the waves' statistics, in wave order
        __shared__ float s_st[2][NW][16];
        if (c4 == 0) {
            s_st[0][wave][j16] = M;
            s_st[1][wave][j16] = S;
        }
        __syncthreads();
        M = s_st[0][0][j16];
#pragma unroll
        for (int w = 1; w < NW; w++) M = fmaxf(M, s_st[0][w][j16]);
        S = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float mw = s_st[0][w][j16];
            S = mw == -INFINITY ? S : fmaf(s_st[1][w][j16], expf(mw - M), S);
        }
    }
    const float inv = 1.0f / S;  // inv = 1 / sum, tensor.rs:304
    // pass 2: the weights times the values
    f4v acc[NT];
#pragma unroll
    for (int q = 0; q < NT; q++) acc[q] = f4v{0.f, 0.f, 0.f, 0.f};
    auto accumulate = [&](int t0, const f4v (&kq)[NQ4], const f4v (&vv)[4][VT]) {
        float s[4];
        scores(t0, kq, s);
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float w = s[r] == -INFINITY ? 0.0f : expf(s[r] - M) * inv;
            p[r] = w < 1e-8f ? 0.0f : w;  // mod.rs:807
        }
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int q = 0; q < NT; q++)
                acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[r], vv[r][q >> 2][q & 3], acc[q], 0, 0, 0);
    };
    {
        f4v ka[NQ4], kb[NQ4], va[4][VT], vb[4][VT];
        load_k(16 * wave, ka);
        load_v(16 * wave, va);
        for (int t0 = 16 * wave; t0 < L; t0 += 2 * STEP) {
            load_k(t0 + STEP, kb);
            load_v(t0 + STEP, vb);
            accumulate(t0, ka, va);
            if (t0 + STEP >= L) break;
            load_k(t0 + 2 * STEP, ka);
            load_v(t0 + 2 * STEP, va);
            accumulate(t0 + STEP, kb, vb);
        }
    }
    // acc[q][i] is column 4 c4 + i, dim 4 j16 + (q & 3) + 64 (q >> 2)
    if constexpr (NW == 1) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int col = 4 * c4 + i, row = r0 + col / gc, head = h0 + col % gc;
            if (col >= rpt * gc || row >= a.n) continue;
            float *o = a.out + ((size_t)row * a.n_head + head) * HD;
#pragma unroll
            for (int v = 0; v < VT; v++)
                *reinterpret_cast<float4 *>(o + 64 * v + 4 * j16) =
                    make_float4(acc[4 * v][i], acc[4 * v + 1][i], acc[4 * v + 2][i], acc[4 * v + 3][i]);
        }
    } else {  // the waves' sums, added in wave order
        __shared__ __align__(16) float s_acc[NW][16][HD];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int v = 0; v < VT; v++)
                *reinterpret_cast<float4 *>(&s_acc[wave][4 * c4 + i][64 * v + 4 * j16]) =
                    make_float4(acc[4 * v][i], acc[4 * v + 1][i], acc[4 * v + 2][i], acc[4 * v + 3][i]);
        __syncthreads();
        for (int i = tid; i < 16 * HD / 4; i += 64 * NW) {
            const int col = i / (HD / 4), d = 4 * (i % (HD / 4)), row = r0 + col / gc, head = h0 + col % gc;
            if (col >= rpt * gc || row >= a.n) continue;
            float4 x = *reinterpret_cast<const float4 *>(&s_acc[0][col][d]);
#pragma unroll
            for (int w = 1; w < NW; w++) {
                const float4 y = *reinterpret_cast<const float4 *>(&s_acc[w][col][d]);
                x = make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
            }
            *reinterpret_cast<float4 *>(a.out + ((size_t)row * a.n_head + head) * HD + d) = x;
        }
    }
}

// P = 16 R nw positions per workgroup of nw waves: four waves with R in
// {1, 2, 4} (hd 64) or {1, 2} (hd 128), or eight waves with R in {1, 2} (hd 64)
// or 1 (hd 128) for P >= 128; the fused-RoPE form when the rope argument is set.
template <int HD, bool ROPE, bool ROWS>
void launch_split_r(const AttnArgs &a, dim3 grid, hipStream_t stream) {
    const int r = a.P / (16 * a.nw);
    const dim3 block(64 * a.nw);
    const unsigned gg = (unsigned)a.group | (unsigned)a.gc << 15 | (a.plus_one ? 1u << 31 : 0u);
#define KH_SPLIT(HH, RR, NN)                                                                                  \
    hipLaunchKernelGGL((attn_split_kernel<HH, RR, NN, ROPE, ROWS>), grid, block, 0, stream, a.len_dev, a.k, a.v, \
                       a.q, (unsigned)a.kstride, (unsigned)a.vstride, a.L, gg, a)
    if (a.nw == 2) {
        KH_SPLIT(HD, 1, 2);
    } else if (a.nw == 8) {
        if (r == 1) KH_SPLIT(HD, 1, 8);
        else KH_SPLIT(64, 2, 8);
    } else if (r == 1) {
        KH_SPLIT(HD, 1, 4);
    } else if (HD == 128 || r == 2) {
        KH_SPLIT(HD, 2, 4);
    } else {
        KH_SPLIT(64, 4, 4);
    }
#undef KH_SPLIT
}

template <int HD>
void launch_split(const AttnArgs &a, dim3 grid, hipStream_t stream) {
    // the row table, or fields too wide for the preloaded words: from the struct
    const bool rows = a.rows || a.kstride > 0x7fffffffu || a.vstride > 0x7fffffffu || a.group > 0x7fff ||
                      a.gc > 0x7fff;
    if (a.rope.kraw) {
        if (rows) launch_split_r<HD, true, true>(a, grid, stream);
        else launch_split_r<HD, true, false>(a, grid, stream);
    } else {
        if (rows) launch_split_r<HD, false, true>(a, grid, stream);
        else launch_split_r<HD, false, false>(a, grid, stream);
    }
}

}  // namespace

namespace {

// The longest sequence taken as one split (every load of the sequence in
// flight in one workgroup): 256 positions at hd 64, 128 at hd 128, as
// measured against split + merge on the box; KVAD_ATTN_SINGLE lowers it
// (0: always split and merge).
size_t single_max(int head_dim) {
    const size_t hw = head_dim == 64 ? 256 : 128;
    const int v = env_int("KVAD_ATTN_SINGLE", -1);
    return v < 0 ? hw : std::min(hw, (size_t)v);
}

// The longest single sequence split into 32-position splits.
size_t short_split_max(int head_dim) { return head_dim == 64 ? 1024 : 512; }

// Query heads per workgroup: the largest divisor of the group size that
// fits the 16 columns of the score product.
int heads_per_wg(int group) {
    int gc = 1;
    for (int c = 1; c <= 16; c++)
        if (group % c == 0) gc = c;
    return gc;
}

// The launch for n_positions (or, with a device length, for at most that
// many): split size, partial buffers carved from ws.
int setup(kh_ctx *ctx, AttnArgs &a, int n_head, int n_kv_head, int head_dim, const float *q, const float *k,
          const float *v, size_t kstride, size_t vstride, size_t n_positions, float *out, int nb = 1) {
    if (n_kv_head <= 0 || n_head <= 0 || n_head % n_kv_head != 0)
        return fail(KH_EINVAL, "attend: n_head must be a positive multiple of n_kv_head");
    if (head_dim != 64 && head_dim != 128)
        return fail(KH_DECLINED, "attend: head_dim other than 64 or 128 runs on the CPU");
    // 32-bit buffer offsets, including a split's overhang past the last row
    if ((n_positions + 256) * kstride * 4 >= 0xffffffffull || (n_positions + 256) * vstride * 4 >= 0xffffffffull)
        return fail(KH_DECLINED, "attend: caches of 4 GiB or more per layer are not addressed here");
    a = AttnArgs{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.kstride = kstride;
    a.vstride = vstride;
    a.n_head = n_head;
    a.group = n_head / n_kv_head;
    const int gc = heads_per_wg(a.group);
    a.gc = gc;
    const int n_hg = n_head / gc;
    a.L = (int)n_positions;
    a.scale = 1.0f / sqrtf((float)head_dim);  // mod.rs:777
    a.out = out;
    // A short sequence runs as one split: the split kernel applies the
    // reference's exact weights itself and no merge is launched.
    if (n_positions <= single_max(head_dim)) {
        int P = 64;
        while ((size_t)P < n_positions) P *= 2;
        a.P = P;
        a.nw = P == 256 ? 8 : 4;
        a.nsplit = 1;
        return KH_OK;
    }
    // positions per split: the largest rung that still gives a workgroup
    // per CU, or a larger one when the merge's split limit needs it
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const int rungs = head_dim == 64 ? 3 : 2;
    const int ladder[3] = {64, 128, 256};
    int step = rungs - 1;
    while (step > 0 && (long long)((n_positions + ladder[step] - 1) / ladder[step]) * n_hg * nb < cu) step--;
    const int forced = env_int("KVAD_ATTN_SPLIT", 0);  // tuning knob: positions per split (32 .. 256)
    for (int i = 0; i < rungs; i++)
        if (ladder[i] == forced) step = i;
    // short sequences past one split: 32 positions on two waves, twice the
    // workgroups (measured: Qwen geometry L = 1024 9.78 -> 9.52 us per layer,
    // Llama-8B L = 512 11.93 -> 11.54; from 2048 positions they lose)
    // (the workspaces size 32-position splits only up to short_split_max, so
    // the knob is honoured only there)
    if (n_positions <= short_split_max(head_dim) && (forced == 32 || (forced == 0 && nb == 1))) {
        a.P = 32;
        a.nw = 2;
        a.nsplit = (int)((n_positions + 31) / 32);
        return KH_OK;
    }
    while (step < rungs - 1 && (n_positions + ladder[step] - 1) / ladder[step] > (size_t)MAX_SPLITS) step++;
    const int P = ladder[step];
    if ((n_positions + P - 1) / P > (size_t)MAX_SPLITS)
        return fail(KH_DECLINED, "attend: sequence longer than the split merge takes");
    a.P = P;
    // waves per workgroup: eight at 256 positions (measured faster at long
    // context), else four; KVAD_ATTN_WAVES = 4 or 8 forces it where P >= 128
    const int fw = env_int("KVAD_ATTN_WAVES", 0);
    a.nw = P >= 128 && (fw == 8 || (fw != 4 && P == 256)) ? 8 : 4;
    a.nsplit = (int)((n_positions + P - 1) / P);
    return KH_OK;
}

// Partials of nsplit splits: pm, pl, pmin [ns], acc [ns][hd], scores [ns][P],
// each array on a 64-byte boundary (hd and P are multiples of 16).
size_t partial_floats(size_t nsplit, int n_head, int head_dim, int P) {
    const size_t ns = nsplit * (size_t)n_head, ns16 = (ns + 15) & ~(size_t)15;
    return 3 * ns16 + ns * (size_t)head_dim + ns * (size_t)P;
}

template <typename Args>
void carve_partials(Args &a, void *ws, int head_dim) {
    const size_t ns = (size_t)a.nsplit * a.n_head, ns16 = (ns + 15) & ~(size_t)15;
    float *p = static_cast<float *>(ws);
    a.pm = p, p += ns16;
    a.pl = p, p += ns16;
    a.pmin = p, p += ns16;
    a.pacc = p, p += ns * head_dim;
    a.psc = p;
}

int run(kh_ctx *ctx, const AttnArgs &a, int head_dim, int nb = 1) {
    dim3 grid(a.nsplit, a.n_head / a.gc, nb);
    if (head_dim == 64) launch_split<64>(a, grid, ctx->stream);
    else launch_split<128>(a, grid, ctx->stream);
    KH_HIP(hipGetLastError());
    if (a.nsplit > 1) {
        const dim3 mg(a.n_head, 1, nb);
        const unsigned pn = (unsigned)a.P | (a.plus_one ? 1u << 31 : 0u);
        const unsigned hg = (unsigned)a.n_head | (unsigned)a.group << 16;
        const bool rows = a.rows || a.n_head > 0xffff || a.group > 0xffff;
#define KH_MERGE(HH, RW)                                                                                           \
    hipLaunchKernelGGL((attn_merge_kernel<HH, RW>), mg, dim3(256), 0, ctx->stream, a.len_dev, a.pm, a.pl, a.pmin, \
                       a.pacc, a.L, pn, hg, a)
        if (head_dim == 64) {
            if (rows) KH_MERGE(64, true);
            else KH_MERGE(64, false);
        } else {
            if (rows) KH_MERGE(128, true);
            else KH_MERGE(128, false);
        }
#undef KH_MERGE
        KH_HIP(hipGetLastError());
    }
    return KH_OK;
}

}  // namespace

size_t attend_single_max(int head_dim) { return head_dim == 64 || head_dim == 128 ? single_max(head_dim) : 0; }

size_t attend_ws_bytes(int n_head, int n_kv_head, int head_dim, size_t max_positions) {
    (void)n_kv_head;
    // splits of 64 or more, or of 32 up to short_split_max: the smallest
    // bounds the count; scores take P per split
    const size_t nsplit = (max_positions + 63) / 64;
    size_t f = partial_floats(nsplit, n_head, head_dim, 64);
    const size_t n32 = (std::min(max_positions, short_split_max(head_dim)) + 31) / 32;
    f = std::max(f, partial_floats(n32, n_head, head_dim, 32));
    return 4 * f + 4 * (max_positions + 256) * (size_t)n_head + 1024;
}

size_t attend_rows_ws_bytes(int n_head, int head_dim, size_t max_positions, size_t nb) {
    // per row as attend_ws_bytes: any split size the launch picks fits
    const size_t nsplit = (max_positions + 63) / 64;
    size_t f = partial_floats(nsplit, n_head, head_dim, 64);
    const size_t n32 = (std::min(max_positions, short_split_max(head_dim)) + 31) / 32;
    f = std::max(f, partial_floats(n32, n_head, head_dim, 32));
    return 4 * nb * (f + (max_positions + 256) * (size_t)n_head) + 1024;
}

size_t attend_rows_need_bytes(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, size_t max_positions,
                              size_t nb) {
    AttnArgs a;
    if (nb == 0 || nb > 65535 || max_positions == 0 ||
        setup(ctx, a, n_head, n_kv_head, head_dim, nullptr, nullptr, nullptr, 0, 0, max_positions, nullptr, (int)nb))
        return 0;
    return 4 * partial_floats(a.nsplit, n_head, head_dim, a.P) * nb + 1024;
}

int launch_attend_rows(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const AttnRow *rows,
                       int nb, size_t kstride, size_t vstride, size_t max_positions, float *out, void *ws,
                       size_t ws_bytes, const AttnRope *rope) {
    if (nb <= 0 || nb > 65535 || max_positions == 0) return fail(KH_EINVAL, "attend: no rows or no positions");
    AttnArgs a;
    int rc = setup(ctx, a, n_head, n_kv_head, head_dim, q, nullptr, nullptr, kstride, vstride, max_positions, out, nb);
    if (rc) return rc;
    a.rows = rows;
    if (rope) a.rope = *rope;
    a.row_floats = partial_floats(a.nsplit, n_head, head_dim, a.P);
    if (4 * a.row_floats * nb > ws_bytes) return fail(KH_EINVAL, "attend: workspace too small for the rows");
    carve_partials(a, ws, head_dim);
    return run(ctx, a, head_dim, nb);
}

// The loads of a pass reach 16 (2 NW + 1) - 1 positions past the longest row.
constexpr size_t PASS_OVERREACH = 16 * (2 * 8 + 1);

bool attend_pass_fits(int head_dim, size_t kstride, size_t vstride, size_t max_positions) {
    if (env_int("KVAD_PASS_ATTN", 1) == 0) return false;
    return (head_dim == 64 || head_dim == 128) && (max_positions + PASS_OVERREACH) * kstride * 4 < 0xffffffffull &&
           (max_positions + PASS_OVERREACH) * vstride * 4 < 0xffffffffull;
}

// Waves per workgroup of a pass: doubled from one while the grid holds
// fewer than two waves per SIMD (2048) and each wave keeps at least four
// 16-position tiles of the longest row; KVAD_PASS_WAVES (1, 2, 4, 8) fixes it.
int pass_waves(int workgroups, size_t max_positions) {
    const int forced = env_int("KVAD_PASS_WAVES", 0);
    if (forced == 1 || forced == 2 || forced == 4 || forced == 8) return forced;
    int nw = 1;
    while (nw < 8 && (size_t)workgroups * nw < 2048 && (size_t)nw * 2 * 64 <= max_positions) nw *= 2;
    return nw;
}

template <int HD>
void launch_pass(kh_ctx *ctx, int nw, dim3 grid, const PassArgs &a) {
    switch (nw) {
        case 1: hipLaunchKernelGGL((attn_pass_kernel<HD, 1>), grid, dim3(64), 0, ctx->stream, a); break;
        case 2: hipLaunchKernelGGL((attn_pass_kernel<HD, 2>), grid, dim3(128), 0, ctx->stream, a); break;
        case 4: hipLaunchKernelGGL((attn_pass_kernel<HD, 4>), grid, dim3(256), 0, ctx->stream, a); break;
        default: hipLaunchKernelGGL((attn_pass_kernel<HD, 8>), grid, dim3(512), 0, ctx->stream, a); break;
    }
}

int launch_attend_pass(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const AttnRow *rows,
                       int n, size_t kstride, size_t vstride, size_t max_positions, float *out) {
    if (n <= 0 || n_kv_head <= 0 || n_head <= 0 || n_head % n_kv_head != 0)
        return fail(KH_EINVAL, "attend_pass: bad row or head count");
    if (!attend_pass_fits(head_dim, kstride, vstride, max_positions))
        return fail(KH_DECLINED, "attend_pass: head_dim 64 or 128 and caches under 4 GiB per layer");
    PassArgs a{};
    a.q = q;
    a.rows = rows;
    a.out = out;
    a.kstride = kstride;
    a.vstride = vstride;
    a.n = n;
    a.n_head = n_head;
    a.group = n_head / n_kv_head;
    a.gc = heads_per_wg(a.group);
    a.scale = 1.0f / sqrtf((float)head_dim);  // mod.rs:777
    const int rpt = 16 / a.gc;
    const dim3 grid((unsigned)((n + rpt - 1) / rpt), (unsigned)(n_head / a.gc));
    if (grid.y > 65535) return fail(KH_EINVAL, "attend_pass: too many head groups");
    const int nw = pass_waves((int)(grid.x * grid.y), max_positions);
    if (head_dim == 64) launch_pass<64>(ctx, nw, grid, a);
    else launch_pass<128>(ctx, nw, grid, a);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int launch_rope_push_rows(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, float *q, const float *k,
                          const float *v, const AttnRow *rows, int nb, size_t kstride, size_t vstride,
                          const AttnRope &rope) {
    if (nb <= 0 || nb > 65535 || n_head <= 0 || n_kv_head <= 0 || n_head + n_kv_head > 65535)
        return fail(KH_EINVAL, "rope_push_rows: bad row or head count");
    const dim3 grid((unsigned)(n_head + n_kv_head), (unsigned)nb);
    if (head_dim == 64)
        hipLaunchKernelGGL(rope_push_rows_kernel<64>, grid, dim3(64), 0, ctx->stream, q, k, v, rows, rope, n_head,
                           n_kv_head, kstride, vstride);
    else if (head_dim == 128)
        hipLaunchKernelGGL(rope_push_rows_kernel<128>, grid, dim3(64), 0, ctx->stream, q, k, v, rows, rope, n_head,
                           n_kv_head, kstride, vstride);
    else
        return fail(KH_DECLINED, "rope_push_rows: head_dim 64 or 128");
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int launch_attend(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const float *k,
                  const float *v, size_t kstride, size_t vstride, size_t n_positions, float *out) {
    if (n_positions == 0) {
        if (n_kv_head <= 0 || n_head <= 0 || n_head % n_kv_head != 0)
            return fail(KH_EINVAL, "attend: n_head must be a positive multiple of n_kv_head");
        return launch_fill(ctx, out, (size_t)n_head * head_dim, 0.0f);
    }
    AttnArgs a;
    int rc = setup(ctx, a, n_head, n_kv_head, head_dim, q, k, v, kstride, vstride, n_positions, out);
    if (rc) return rc;
    if (a.nsplit > 1) {
        if ((rc = ensure(ctx, ctx->ws, 4 * partial_floats(a.nsplit, n_head, head_dim, a.P) + 1024))) return rc;
        carve_partials(a, ctx->ws.ptr, head_dim);
    }
    return run(ctx, a, head_dim);
}

// ---------------------------------------------------------------------------
// Attention for callers that cannot allocate (graph capture, tight serving
// loops): the split partials live in `scratch`, a static device array of
// SCRATCH_BYTES per GPU, held from library load until the process ends.
// Host code never uses the array's name as an address: scratch_init looks up
// the device address once per device, with that device current, and the
// launches take that pointer.  Every call on a device shares its array, so
// calls that overlap on one GPU (two streams, two threads) race; calls on one
// stream are ordered.  Nothing in it has to start at zero: the split kernel
// writes every partial the merge reads.
// ---------------------------------------------------------------------------
constexpr size_t SCRATCH_BYTES = 8u << 20;
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];
namespace {
constexpr int SCRATCH_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch[SCRATCH_DEVICES];  // per device: the array's device address
}  // namespace

int scratch_init(int device) {
    if (device < 0 || device >= SCRATCH_DEVICES) return fail(KH_EINVAL, "scratch: device index out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch[device]) return KH_OK;
    int cur = -1;
    KH_HIP(hipGetDevice(&cur));
    if (cur != device) return fail(KH_EINVAL, "scratch: set up with another device current");
    void *p = nullptr;
    KH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(KH_EHIP, "scratch: no device address for the scratch array");
    g_scratch[device] = p;
    return KH_OK;
}

size_t scratch_bytes() { return SCRATCH_BYTES; }

int launch_attend_noalloc(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const float *k,
                          const float *v, size_t kstride, size_t vstride, size_t n_positions, float *out) {
    void *ws = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        if (ctx->device >= 0 && ctx->device < SCRATCH_DEVICES) ws = g_scratch[ctx->device];
    }
    if (!ws) return fail(KH_EINVAL, "attend_noalloc: this device's scratch array was not set up by kh_init");
    if (n_positions == 0) {
        if (n_kv_head <= 0 || n_head <= 0 || n_head % n_kv_head != 0)
            return fail(KH_EINVAL, "attend: n_head must be a positive multiple of n_kv_head");
        return launch_fill(ctx, out, (size_t)n_head * head_dim, 0.0f);
    }
    AttnArgs a;
    int rc = setup(ctx, a, n_head, n_kv_head, head_dim, q, k, v, kstride, vstride, n_positions, out);
    if (rc) return rc;
    if (a.nsplit > 1) {
        const size_t need = 4 * partial_floats(a.nsplit, n_head, head_dim, a.P) + 1024;
        if (need > SCRATCH_BYTES)
            return fail(KH_EINVAL, "attend_noalloc: this call needs " + std::to_string(need) +
                                       " bytes of scratch, more than the " + std::to_string(SCRATCH_BYTES) +
                                       " the library holds per device");
        carve_partials(a, ws, head_dim);
    }
    return run(ctx, a, head_dim);
}

int launch_attend_devlen(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const float *k,
                         const float *v, size_t kstride, size_t vstride, const int32_t *len_dev, int plus_one,
                         size_t max_positions, float *out, void *ws, size_t ws_bytes, const AttnRope *rope) {
    if (max_positions == 0) return fail(KH_EINVAL, "attend: no positions");
    AttnArgs a;
    int rc = setup(ctx, a, n_head, n_kv_head, head_dim, q, k, v, kstride, vstride, max_positions, out);
    if (rc) return rc;
    if (4 * partial_floats(a.nsplit, n_head, head_dim, a.P) > ws_bytes)
        return fail(KH_EINVAL, "attend: workspace too small for the launch");
    a.len_dev = len_dev;
    a.plus_one = plus_one;
    if (rope) {  // the caches are written at the new position
        a.rope = *rope;
        a.kw = const_cast<float *>(k);
        a.vw = const_cast<float *>(v);
    }
    carve_partials(a, ws, head_dim);
    return run(ctx, a, head_dim);
}


// ---------------------------------------------------------------------------
// Latent attention, absorbed (model/deepseek.rs:553-591): every query head
// scores the same cached row [c_t (512) | pe_t (64)] with [q_lat_h | q_pe_h]
// and averages the compressed rows c_t -- GQA with one shared "KV head" of
// key width 576 and value width 512, so a workgroup takes up to 16 heads, the
// 16 columns of the score product, with no padding at DeepSeek's 16.
// ---------------------------------------------------------------------------
namespace {

constexpr int MLA_LAT = 512, MLA_ROPE = 64, MLA_K = MLA_LAT + MLA_ROPE;
constexpr int MLA_QSTR = MLA_K + 4;  // LDS row stride (floats) of the staged queries
constexpr int MLA_P = 64;            // positions per workgroup: one tile of 16 per wave
// dims per merge workgroup: 128 (four per head) for a few splits, 64 from
// 64 splits on, where each workgroup's partials are what it waits for
// (measured at L = 1024 / 8192 / 32768: 18.9 / 24.6 / 44.2 us per layer at
// 128, 19.0 / 24.3 / 42.8 at 64, 19.4 / 24.8 / 43.0 at 32)
int mla_merge_dims(int nsplit) {
    const int forced = env_int("KVAD_MLA_MERGE_D", 0);  // tuning knob: 32, 64 or 128
    if (forced == 32 || forced == 64 || forced == 128) return forced;
    return nsplit >= 64 ? 64 : 128;
}

struct MlaArgs {
    const float *q_lat, *q_pe;  // [n_head][512], [n_head][64]
    const float *c, *pe;        // cached rows: c [L][cstride], pe [L][pestride]
    size_t cstride, pestride;
    int n_head, L, nsplit;
    float scale;
    float *pm, *pl, *pmin, *pacc, *psc;  // per split: [nsplit][n_head]; acc [..][512]; scores [..][P]
    float *out;                    // [n_head][512]
    int P;                         // positions per split: 16 per wave
};

// Split kernel.  Wave w scores positions t0 + 16w .. +15 for the 16 heads:
// S = K' Q'^T on v_mfma_f32_16x16x4_f32 over 36 products of 16 dims (32 of
// c, 4 of pe, so each reads one array); in product 4k + i k-slot c takes
// dims 64k + 16i + 4c .. + 3, so one load instruction reads 64 contiguous
// bytes of each row.  Lane (c, j) holds 144 dims of its row, all loads in
// flight at once; the queries sit in LDS, dealt the same way.
// The workgroup takes one maximum per head, so every wave's exponentials
// share it; the probabilities go to LDS and wave w then forms
// O[heads][dims 128w .. 128w + 127] = P V over all 64 positions.
template <int NW>
__global__ __launch_bounds__(64 * NW) void mla_split_kernel(MlaArgs a) {
    constexpr int P = 16 * NW;       // positions: one tile of 16 per wave
    constexpr int DW = MLA_LAT / NW;  // value dims each wave forms
    constexpr int VG = DW / 64;       // 64-dim groups of them
    const int split = blockIdx.x, h0 = blockIdx.y * 16;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j16 = lane & 15, c4 = lane >> 4;
    const int L = a.L;
    const int t0 = split * P, n = min(L - t0, P);
    const bool whole = a.nsplit == 1;
    const int H = min(a.n_head - h0, 16);
    __shared__ __align__(16) float sQ[16 * MLA_QSTR];
    __shared__ float sP[16][P + 4];
    __shared__ float s_st[3][NW][16];
    const rsrc_t C = rsrc(a.c, (size_t)L * a.cstride * 4), PE = rsrc(a.pe, (size_t)L * a.pestride * 4);

    // the tile's key rows (the long-latency loads) first
    f4v kq[9][4];
    {
        const size_t pos = (size_t)(t0 + 16 * wave + j16);
        // lane (c4, j16), load (k, i): dims 64 k + 16 i + 4 c4 .. + 3, so each
        // load instruction reads 64 contiguous bytes of every row
        const unsigned off = (unsigned)((pos * a.cstride + 4 * c4) * 4);
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                kq[k][i] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(C, off, 256 * k + 64 * i, 0));
        const unsigned poff = (unsigned)((pos * a.pestride + 4 * c4) * 4);
#pragma unroll
        for (int i = 0; i < 4; i++)
            kq[8][i] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(PE, poff, 64 * i, 0));
    }
    // the queries [q_lat | q_pe] of the group's heads, zero rows past H
    for (int i = tid; i < 16 * (MLA_K / 4); i += 64 * NW) {
        const int h = i / (MLA_K / 4), d4 = i % (MLA_K / 4);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (h < H)
            v = d4 < MLA_LAT / 4
                    ? *reinterpret_cast<const float4 *>(a.q_lat + (size_t)(h0 + h) * MLA_LAT + 4 * d4)
                    : *reinterpret_cast<const float4 *>(a.q_pe + (size_t)(h0 + h) * MLA_ROPE + 4 * (d4 - MLA_LAT / 4));
        *reinterpret_cast<float4 *>(&sQ[h * MLA_QSTR + 4 * d4]) = v;
    }
    __syncthreads();

    // scores: lane (c4, j16) ends with positions 4 c4 .. 4 c4 + 3 of the tile, head j16
    f4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 9; k++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const f4v q4 = *reinterpret_cast<const f4v *>(&sQ[j16 * MLA_QSTR + 64 * k + 16 * i + 4 * c4]);
#pragma unroll
            for (int e = 0; e < 4; e++) d = __builtin_amdgcn_mfma_f32_16x16x4f32(kq[k][i][e], q4[e], d, 0, 0, 0);
        }
    // The value rows (the latent c again, in the P V operand layout), every
    // load issued now, before the softmax's reductions and barriers: left to
    // itself the scheduler streams them after the barriers, two at a time
    // with a wait between.
    const int D0 = DW * wave;
    f4v vv[NW][4][VG];
#pragma unroll
    for (int u = 0; u < NW; u++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const size_t p = (size_t)(t0 + 16 * u + 4 * c4 + r);
            const unsigned off = (unsigned)((p * a.cstride + D0 + 4 * j16) * 4);
#pragma unroll
            for (int v = 0; v < VG; v++)
                vv[u][r][v] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(C, off, 256 * v, 0));
        }
    __builtin_amdgcn_sched_barrier(0);
    float s[4], mx = -INFINITY, mn = INFINITY;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const bool ok = j16 < H && 16 * wave + 4 * c4 + r < n;
        const float sc = d[r] * a.scale;  // (dot(q_lat, c) + dot(q_pe, pe)) * scale, deepseek.rs:567-570
        s[r] = ok ? sc : -INFINITY;
        mx = fmaxf(mx, s[r]);
        mn = ok ? fminf(mn, sc) : mn;
    }
    mx = rows_max(mx);
    mn = rows_min(mn);
    if (c4 == 0) {
        s_st[0][wave][j16] = mx;
        s_st[2][wave][j16] = mn;
    }
    __syncthreads();
    auto wmax = [&](int st, int h) {
        float x = s_st[st][0][h];
#pragma unroll
        for (int w = 1; w < NW; w++) x = fmaxf(x, s_st[st][w][h]);
        return x;
    };
    auto wsum = [&](int h) {  // in wave order
        float x = s_st[1][0][h];
#pragma unroll
        for (int w = 1; w < NW; w++) x = x + s_st[1][w][h];
        return x;
    };
    const float M = wmax(0, j16);
    float e[4], l = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        e[r] = s[r] == -INFINITY ? 0.0f : expf(s[r] - M);
        l += e[r];
    }
    l = rows_sum(l);
    if (c4 == 0) s_st[1][wave][j16] = l;
    __syncthreads();
    const float S = wsum(j16);
    if (whole) {
        // the reference's own weights: w = exp(s - M) * (1/S), dropping w < 1e-8
        // (softmax_inplace, tensor.rs:297-308; deepseek.rs:576-579)
        const float inv = 1.0f / S;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float w = e[r] * inv;
            e[r] = w < 1e-8f ? 0.0f : w;
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) sP[j16][16 * wave + 4 * c4 + r] = e[r];
    __syncthreads();

    // values: wave w forms dims DW w .. DW w + DW - 1 for every position of
    // the split (their loads were issued after the scores)
    f4v acc[4 * VG];
#pragma unroll
    for (int q = 0; q < 4 * VG; q++) acc[q] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NW; u++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float pa = sP[j16][16 * u + 4 * c4 + r];  // head j16, position 4 c4 + r of tile u
#pragma unroll
            for (int v = 0; v < VG; v++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    acc[4 * v + q] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, vv[u][r][v][q], acc[4 * v + q], 0, 0, 0);
        }
    // acc[4 v + q][i]: head 4 c4 + i, dim D0 + 64 v + 4 j16 + q
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int h = 4 * c4 + i;
        if (h >= H) continue;
        float *dst = whole ? a.out + (size_t)(h0 + h) * MLA_LAT
                           : a.pacc + ((size_t)split * a.n_head + h0 + h) * MLA_LAT;
#pragma unroll
        for (int v = 0; v < VG; v++)
            *reinterpret_cast<float4 *>(dst + D0 + 64 * v + 4 * j16) =
                make_float4(acc[4 * v][i], acc[4 * v + 1][i], acc[4 * v + 2][i], acc[4 * v + 3][i]);
    }
    if (!whole && tid < H) {
        const int h = tid;
        const size_t o = (size_t)split * a.n_head + h0 + h;
        a.pm[o] = wmax(0, h);
        a.pl[o] = wsum(h);
        float mnv = s_st[2][0][h];
#pragma unroll
        for (int w = 1; w < NW; w++) mnv = fminf(mnv, s_st[2][w][h]);
        a.pmin[o] = mnv;
    }
    if (!whole && j16 < H)  // the scores, for the merge's decision on the 1e-8 skip (stored last)
        *reinterpret_cast<float4 *>(a.psc + ((size_t)split * a.n_head + h0 + j16) * P + 16 * wave + 4 * c4) =
            make_float4(s[0], s[1], s[2], s[3]);
}

// Merge, one workgroup per head and 128 dims (merge_head): the value row of position t is c_t.
template <int D>
__global__ __launch_bounds__(256) void mla_merge_kernel(MlaArgs a) {
    const int h = blockIdx.x;
    const rsrc_t C = rsrc(a.c, (size_t)a.L * a.cstride * 4);
    auto vrow = [&](int t, int d4) {
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                              C, (unsigned)(((size_t)t * a.cstride + 4 * d4) * 4), 0, 0));
    };
    if (a.nsplit <= merge_fast_max(D) &&
        merge_head_fast<MLA_LAT, D>(a.pm, a.pl, a.pmin, a.pacc, a.nsplit, a.n_head, h, D * blockIdx.y, a.out))
        return;
    merge_head<MLA_LAT, D>(a.pm, a.pl, a.pmin, a.pacc, a.psc, a.nsplit, a.n_head, h, D * blockIdx.y, a.P, a.L,
                           vrow, a.out);
}

}  // namespace

int launch_mla(kh_ctx *ctx, int n_head, const float *q_lat, const float *q_pe, const float *c, const float *pe,
               size_t cstride, size_t pestride, size_t n_positions, float scale, float *out) {
    if (n_head <= 0) return fail(KH_EINVAL, "mla_attend: n_head must be positive");
    if (n_positions == 0) return launch_fill(ctx, out, (size_t)n_head * MLA_LAT, 0.0f);
    if (cstride < MLA_LAT || pestride < MLA_ROPE || cstride % 4 || pestride % 4)
        return fail(KH_EINVAL, "mla_attend: row strides must hold a row and be multiples of 4 floats");
    if ((n_positions + MLA_P) * cstride * 4 >= 0xffffffffull || (n_positions + MLA_P) * pestride * 4 >= 0xffffffffull)
        return fail(KH_DECLINED, "mla_attend: caches of 4 GiB or more per layer are not addressed here");
    MlaArgs a{};
    a.q_lat = q_lat, a.q_pe = q_pe, a.c = c, a.pe = pe, a.cstride = cstride, a.pestride = pestride;
    a.n_head = n_head;
    a.L = (int)n_positions;
    // positions per split: 128 (eight waves) while that still gives a
    // workgroup per CU -- half the partials to write and merge; 32 (two
    // waves) for short sequences past one split, twice the workgroups
    // (measured at L = 1024 / 8192 / 32768: 18.9 / 24.4 / 40.8 us per layer
    // by this rule, 17.7 / 27.2 / 51.0 with 32 everywhere); else 64
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const int hg = (n_head + 15) / 16;
    const int forced = env_int("KVAD_MLA_SPLIT", 0);  // tuning knob: positions per split (32 / 64 / 128)
    a.P = forced == 32 || forced == 64 || forced == 128 ? forced
          : (long long)((n_positions + 127) / 128) * hg >= cu ? 128
          : n_positions > (size_t)MLA_P && n_positions <= 1024 ? 32
                                                               : MLA_P;
    a.nsplit = (int)((n_positions + a.P - 1) / a.P);
    if (a.nsplit > MAX_SPLITS) return fail(KH_DECLINED, "mla_attend: sequence longer than the split merge takes");
    a.scale = scale;
    a.out = out;
    if (a.nsplit > 1) {
        int rc = ensure(ctx, ctx->ws, 4 * partial_floats(a.nsplit, n_head, MLA_LAT, a.P) + 1024);
        if (rc) return rc;
        carve_partials(a, ctx->ws.ptr, MLA_LAT);
    }
    if (a.P == 128)
        hipLaunchKernelGGL((mla_split_kernel<8>), dim3(a.nsplit, hg), dim3(512), 0, ctx->stream, a);
    else if (a.P == 32)
        hipLaunchKernelGGL((mla_split_kernel<2>), dim3(a.nsplit, hg), dim3(128), 0, ctx->stream, a);
    else
        hipLaunchKernelGGL((mla_split_kernel<4>), dim3(a.nsplit, hg), dim3(256), 0, ctx->stream, a);
    KH_HIP(hipGetLastError());
    if (a.nsplit > 1) {
        const int fd = mla_merge_dims(a.nsplit);
        if (fd == 32)
            hipLaunchKernelGGL((mla_merge_kernel<32>), dim3(n_head, MLA_LAT / 32), dim3(256), 0, ctx->stream, a);
        else if (fd == 64)
            hipLaunchKernelGGL((mla_merge_kernel<64>), dim3(n_head, MLA_LAT / 64), dim3(256), 0, ctx->stream, a);
        else
            hipLaunchKernelGGL((mla_merge_kernel<128>), dim3(n_head, MLA_LAT / 128), dim3(256), 0, ctx->stream, a);
        KH_HIP(hipGetLastError());
    }
    return KH_OK;
}

}  // namespace kh
