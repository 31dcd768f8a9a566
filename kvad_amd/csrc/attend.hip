// GQA decode attention over a device-resident KV cache, split along the
// sequence: one launch computes per-split partial softmax sums, a second
// merges them.
//
// Reference: model::attend (crates/llm/src/model/mod.rs:769-819) with
// tensor::dot (tensor.rs:220-235) and softmax_inplace (tensor.rs:297-308).
// The reference walks every cached key once per query head; here a workgroup
// owns one KV head's query heads (up to 8 of them) and a run of P positions,
// and reads each key and value row once for the whole group -- the
// restructuring the reference's notes ask for (docs/engine.md:783-791).
//
// Split kernel, workgroup (split j, head group): all its K and V rows are
// loaded up front (16 lanes per row, 16 rows per pass); scores s = dot(q, k)
// * scale; local max m_j, l_j = sum exp(s - m_j), acc_j = sum exp(s - m_j) v,
// and the smallest score.  When one split covers the whole sequence it
// finishes the job itself with the reference's exact weights
// w = exp(s - M) * (1/S), dropping w < 1e-8 (mod.rs:807).
//
// Merge kernel, one workgroup per query head:
//   M = max m_j,  S = sum l_j exp(m_j - M),  acc = sum exp(m_j - M) acc_j,
// and out = acc * (1/S).  The reference's skip of weights below 1e-8 can
// only bite in a split whose smallest score is below M + ln S + ln 1e-8
// (checked with a margin); such a split's positions are scored again,
// identically, and each skipped term w * v is taken back out.  Real scores
// never qualify (it takes a gap of about 18 + ln S), so the fast path is the
// whole cost; the slow path keeps the reference's weights when it does occur.
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

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

// Sum over each row of 16 lanes; all 16 get it, in a fixed order.
__device__ __forceinline__ float row16_sum(float v) {
    v += dppf<DPP_XOR1>(v);
    v += dppf<DPP_XOR2>(v);
    v += dppf<DPP_HALF_MIRROR>(v);
    v += dppf<DPP_MIRROR>(v);
    return v;
}

__device__ __forceinline__ float lane_read(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dppf<DPP_XOR1>(v));
    v = fmaxf(v, dppf<DPP_XOR2>(v));
    v = fmaxf(v, dppf<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dppf<DPP_MIRROR>(v));
    return fmaxf(fmaxf(lane_read(v, 0), lane_read(v, 16)), fmaxf(lane_read(v, 32), lane_read(v, 48)));
}

__device__ __forceinline__ float wave_min(float v) {
    v = fminf(v, dppf<DPP_XOR1>(v));
    v = fminf(v, dppf<DPP_XOR2>(v));
    v = fminf(v, dppf<DPP_HALF_MIRROR>(v));
    v = fminf(v, dppf<DPP_MIRROR>(v));
    return fminf(fminf(lane_read(v, 0), lane_read(v, 16)), fminf(lane_read(v, 32), lane_read(v, 48)));
}

__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    return (lane_read(v, 0) + lane_read(v, 16)) + (lane_read(v, 32) + lane_read(v, 48));
}

struct AttnArgs {
    const float *q;
    const float *k;
    const float *v;
    size_t kstride, vstride;  // floats between consecutive positions
    size_t kbytes, vbytes;    // readable bytes of the k and v arrays
    int n_head, group, gc;    // group = n_head / n_kv_head; gc = heads per workgroup
    int L, P, nsplit;
    // when set, the length is read here (+ plus_one) and L/nsplit above are
    // the launch's maxima; splits past the length return at once
    const int32_t *len_dev;
    int plus_one;
    float scale;
    // per split, [nsplit][n_head]: local max, sum, smallest score; and acc
    float *pm, *pl, *pmin, *pacc;
    float *out;               // [n_head][hd]
};

// One position's scores for the G heads from the 16-lane row's slices: the
// same arithmetic wherever a score is needed.
template <int GM, int DPL>
__device__ __forceinline__ void score_row(const float (&qr)[GM][DPL], const float (&kv)[DPL], float scale, int G,
                                          float (&s)[GM]) {
#pragma unroll
    for (int h = 0; h < GM; h++) {
        float a = 0.0f;
        if (h < G) {
#pragma unroll
            for (int d = 0; d < DPL; d++) a = fmaf(qr[h][d], kv[d], a);
        }
        a = row16_sum(a);
        s[h] = a * scale;  // dot(q, k) * scale, mod.rs:802
    }
}

template <int DPL>
__device__ __forceinline__ void load_row(const rsrc_t &R, unsigned off, float (&r)[DPL]) {
#pragma unroll
    for (int d = 0; d < DPL; d += 4) {
        const float4 f = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(R, off, d * 4, 0));
        r[d] = f.x, r[d + 1] = f.y, r[d + 2] = f.z, r[d + 3] = f.w;
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
//           heads; k-slot c of lane (c, i) covers the head dims
//           [c HD/4, (c+1) HD/4), one product per dim, so lane (c, i) reads
//           HD bytes of key row i contiguously; the 16 columns are the G
//           query heads (the rest zero).
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

template <int HD, int R>
__global__ __launch_bounds__(256) void attn_split_kernel(AttnArgs a) {
    constexpr int HQ = HD / 4;   // dims per k-slot of the score product
    constexpr int NQ4 = HQ / 4;  // float4s per lane of a key row
    constexpr int VT = HD / 64;  // float4s per lane of a value row
    constexpr int NT = HD / 16;  // 16-column tiles of the output
    constexpr int P = 64 * R;
    const int split = blockIdx.x, hg = blockIdx.y;
    const int G = a.gc;
    const int h0 = hg * G, kvh = h0 / a.group;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j16 = lane & 15, c4 = lane >> 4;
    const int L = a.len_dev ? min(*a.len_dev + a.plus_one, a.L) : a.L;
    const int nsplit = (L + P - 1) / P;
    if (split >= nsplit) return;
    const int t0 = split * P;
    const int n = min(L - t0, P);
    const bool whole = nsplit == 1;
    const rsrc_t K = rsrc(a.k, (size_t)L * a.kstride * 4), V = rsrc(a.v, (size_t)L * a.vstride * 4);
    const int pw = wave * 16 * R;  // the wave's first position in the split

    __shared__ __align__(16) float s_acc[4][16][HD];  // per-wave totals
    __shared__ float s_st[3][4][16];                  // per-wave max, sum, smallest score

    // q first (the score products wait on it before any key), then keys,
    // then values: loads complete in issue order
    const bool hv = j16 < G;
    f4v qb4[NQ4];
    {
        const float *qh = a.q + (size_t)(h0 + (hv ? j16 : 0)) * HD + HQ * c4;
#pragma unroll
        for (int m = 0; m < NQ4; m++) {
            const float4 f = *reinterpret_cast<const float4 *>(qh + 4 * m);
            qb4[m] = hv ? f4v{f.x, f.y, f.z, f.w} : f4v{0.f, 0.f, 0.f, 0.f};
        }
    }
    f4v kq[R][NQ4];
    f4v vv[R][4][VT];
#pragma unroll
    for (int u = 0; u < R; u++) {
        const size_t t = (size_t)(t0 + pw + 16 * u + j16);
        const unsigned off = (unsigned)((t * a.kstride + (size_t)kvh * HD + HQ * c4) * 4);
#pragma unroll
        for (int m = 0; m < NQ4; m++)
            kq[u][m] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(K, off, 16 * m, 0));
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
        for (int i = tid; i < G * HD; i += 256) {
            const int h = i / HD, d = i % HD;
            const float M = fmaxf(fmaxf(s_st[0][0][h], s_st[0][1][h]), fmaxf(s_st[0][2][h], s_st[0][3][h]));
            float x = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float c = s_st[0][w][h] == -INFINITY ? 0.0f : expf(s_st[0][w][h] - M);
                x = fmaf(c, s_acc[w][h][d], x);
            }
            a.pacc[((size_t)split * a.n_head + h0 + h) * HD + d] = x;
        }
        if (tid < G) {
            const int h = tid;
            const float M = fmaxf(fmaxf(s_st[0][0][h], s_st[0][1][h]), fmaxf(s_st[0][2][h], s_st[0][3][h]));
            float Ls = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float c = s_st[0][w][h] == -INFINITY ? 0.0f : expf(s_st[0][w][h] - M);
                Ls = fmaf(c, s_st[1][w][h], Ls);
            }
            const size_t o = (size_t)split * a.n_head + h0 + h;
            a.pm[o] = M;
            a.pl[o] = Ls;
            a.pmin[o] = fminf(fminf(s_st[2][0][h], s_st[2][1][h]), fminf(s_st[2][2][h], s_st[2][3][h]));
        }
        return;
    }

    // One split is the whole sequence: the reference's own weights
    // w = exp(s - M) * (1/S), S = sum exp(s - M), dropping w < 1e-8
    // (softmax_inplace, tensor.rs:297-308; mod.rs:805-812).
    if (c4 == 0 && hv) s_st[0][wave][j16] = mx;
    __syncthreads();
    const int hj = hv ? j16 : 0;
    const float M = fmaxf(fmaxf(s_st[0][0][hj], s_st[0][1][hj]), fmaxf(s_st[0][2][hj], s_st[0][3][hj]));
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
    const float inv = 1.0f / (((s_st[1][0][hj] + s_st[1][1][hj]) + s_st[1][2][hj]) + s_st[1][3][hj]);
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
    for (int i = tid; i < G * HD; i += 256) {
        const int h = i / HD, d = i % HD;
        a.out[(size_t)(h0 + h) * HD + d] = ((s_acc[0][h][d] + s_acc[1][h][d]) + s_acc[2][h][d]) + s_acc[3][h][d];
    }
}

// Fixed-order tree over the 256 threads' values; every thread gets the result.
template <typename F>
__device__ __forceinline__ float block_reduce(float v, float *s_red, F op) {
    const int tid = threadIdx.x;
    s_red[tid] = v;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) s_red[tid] = op(s_red[tid], s_red[tid + w]);
        __syncthreads();
    }
    const float r = s_red[0];
    __syncthreads();
    return r;
}

constexpr int MAX_SPLITS = 4096;

template <int HD>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnArgs a) {
    constexpr int DPL = HD / 16;
    constexpr int NQ = HD / 4, NSG = 256 / NQ;  // float4 slices of a row; split groups
    const int h = blockIdx.x, tid = threadIdx.x;
    const int L = a.len_dev ? min(*a.len_dev + a.plus_one, a.L) : a.L;
    const int ns = (L + a.P - 1) / a.P, n_head = a.n_head;
    if (ns <= 1) return;  // the split kernel finished a single split itself
    __shared__ float s_red[256];
    __shared__ float s_c[MAX_SPLITS];           // exp(m_j - M)
    __shared__ __align__(16) float s_acc[NSG][HD];
    __shared__ float s_fix[16][HD];
    __shared__ int s_need;

    // the splits' statistics, all loads in flight together
    float mx = -INFINITY, lo = INFINITY;
    for (int i = tid; i < ns; i += 256) {
        mx = fmaxf(mx, a.pm[(size_t)i * n_head + h]);
        lo = fminf(lo, a.pmin[(size_t)i * n_head + h]);
    }
    const float M = block_reduce(mx, s_red, [](float x, float y) { return fmaxf(x, y); });
    lo = block_reduce(lo, s_red, [](float x, float y) { return fminf(x, y); });

    // c_j = exp(m_j - M);  S = sum l_j c_j
    float s = 0.0f;
    for (int i = tid; i < ns; i += 256) {
        const size_t o = (size_t)i * n_head + h;
        const float c = expf(a.pm[o] - M);
        s_c[i] = c;
        s = fmaf(a.pl[o], c, s);
    }
    const float S = block_reduce(s, s_red, [](float x, float y) { return x + y; });  // syncs s_c too
    const float inv = 1.0f / S;  // inv = 1 / sum, tensor.rs:304

    // acc[d] = sum_j c_j acc_j[d]: thread (split group sg, float4 slice dq)
    // walks splits sg, sg + NSG, ... eight loads at a time
    {
        const int sg = tid / NQ, dq = tid % NQ;
        const rsrc_t PA = rsrc(a.pacc, (size_t)ns * n_head * HD * 4);
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int i0 = sg; i0 < ns; i0 += 8 * NSG) {
            float4 v[8];
            float c[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = i0 + u * NSG;
                v[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      PA, (unsigned)((((size_t)i * n_head + h) * HD + 4 * dq) * 4), 0, 0));
                c[u] = i < ns ? s_c[i] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                x.x = fmaf(c[u], v[u].x, x.x);
                x.y = fmaf(c[u], v[u].y, x.y);
                x.z = fmaf(c[u], v[u].z, x.z);
                x.w = fmaf(c[u], v[u].w, x.w);
            }
        }
        *reinterpret_cast<float4 *>(&s_acc[sg][4 * dq]) = x;
    }
    __syncthreads();

    // ---- skip correction: w = exp(s - M) * (1/S) < 1e-8 ---------------------
    // possible only where a score is below M + ln S + ln 1e-8 (with a margin)
    const float thr = M + logf(S) - 18.420681f + 1.0f;
    if (lo < thr) {
        const int group16 = tid >> 4, sub = tid & 15, kvh = h / a.group;
        const rsrc_t K = rsrc(a.k, (size_t)L * a.kstride * 4), V = rsrc(a.v, (size_t)L * a.vstride * 4);
        float qr[1][DPL];
#pragma unroll
        for (int d = 0; d < DPL; d++) qr[0][d] = a.q[(size_t)h * HD + sub * DPL + d];
        float fix[DPL];
#pragma unroll
        for (int d = 0; d < DPL; d++) fix[d] = 0.0f;
        for (int j = 0; j < ns; j++) {
            if (tid == 0) s_need = a.pmin[(size_t)j * n_head + h] < thr;
            __syncthreads();
            const int need = s_need;
            __syncthreads();
            if (!need) continue;
            const int tj = j * a.P, nj = min(L - tj, a.P);
            for (int base = 0; base < nj; base += 16) {
                const int t = tj + base + group16;
                if (base + group16 >= nj) continue;  // whole 16-lane rows drop out together
                float kv[DPL], vv[DPL];
                load_row<DPL>(K, (unsigned)(((size_t)t * a.kstride + (size_t)kvh * HD + sub * DPL) * 4), kv);
                load_row<DPL>(V, (unsigned)(((size_t)t * a.vstride + (size_t)kvh * HD + sub * DPL) * 4), vv);
                float sc[1];
                score_row<1, DPL>(qr, kv, a.scale, 1, sc);
                float w = expf(sc[0] - M);
                w = w * inv;
                if (w < 1e-8f) {
#pragma unroll
                    for (int d = 0; d < DPL; d++) fix[d] = fmaf(w, vv[d], fix[d]);
                }
            }
        }
#pragma unroll
        for (int d = 0; d < DPL; d++) s_fix[group16][sub * DPL + d] = fix[d];
        __syncthreads();
        if (tid < HD) {
            float f = 0.0f;
            for (int g = 0; g < 16; g++) f += s_fix[g][tid];
            s_fix[0][tid] = f;
        }
        __syncthreads();
    }
    if (tid < HD) {
        float x = s_acc[0][tid];
#pragma unroll
        for (int g = 1; g < NSG; g++) x += s_acc[g][tid];
        x = x * inv;
        if (lo < thr) x -= s_fix[0][tid];
        a.out[(size_t)h * HD + tid] = x;
    }
}

// P = 64 R positions per workgroup: R in {1, 2, 4} for hd 64, {1, 2} for hd 128.
template <int HD>
void launch_split(const AttnArgs &a, dim3 grid, hipStream_t stream) {
    const int r = a.P / 64;
    if (r == 1) hipLaunchKernelGGL((attn_split_kernel<HD, 1>), grid, dim3(256), 0, stream, a);
    else if (HD == 128 || r == 2) hipLaunchKernelGGL((attn_split_kernel<HD, 2>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((attn_split_kernel<64, 4>), grid, dim3(256), 0, stream, a);
}

}  // namespace

namespace {

// The launch for n_positions (or, with a device length, for at most that
// many): split size, partial buffers carved from ws.
int setup(kh_ctx *ctx, AttnArgs &a, int n_head, int n_kv_head, int head_dim, const float *q, const float *k,
          const float *v, size_t kstride, size_t vstride, size_t n_positions, float *out) {
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
    a.kbytes = n_positions * kstride * 4;
    a.vbytes = n_positions * vstride * 4;
    a.n_head = n_head;
    a.group = n_head / n_kv_head;
    int gc = 1;  // query heads per workgroup: the 16 columns of the score product
    for (int c = 1; c <= 16; c++)
        if (a.group % c == 0) gc = c;
    a.gc = gc;
    const int n_hg = n_head / gc;
    a.L = (int)n_positions;
    // positions per split: the largest rung that still gives a workgroup
    // per CU, or a larger one when the merge's split limit needs it
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const int rungs = head_dim == 64 ? 3 : 2;
    const int ladder[3] = {64, 128, 256};
    int step = rungs - 1;
    while (step > 0 && (long long)((n_positions + ladder[step] - 1) / ladder[step]) * n_hg < cu) step--;
    while (step < rungs - 1 && (n_positions + ladder[step] - 1) / ladder[step] > (size_t)MAX_SPLITS) step++;
    const int P = ladder[step];
    if ((n_positions + P - 1) / P > (size_t)MAX_SPLITS)
        return fail(KH_DECLINED, "attend: sequence longer than the split merge takes");
    a.P = P;
    a.nsplit = (int)((n_positions + P - 1) / P);
    a.scale = 1.0f / sqrtf((float)head_dim);  // mod.rs:777
    a.out = out;
    return KH_OK;
}

void carve(AttnArgs &a, void *ws, int head_dim) {
    const size_t ns = (size_t)a.nsplit * a.n_head;
    float *p = static_cast<float *>(ws);
    a.pm = p, p += ns;
    a.pl = p, p += ns;
    a.pmin = p, p += ns;
    a.pacc = p;
    (void)head_dim;
}

int run(kh_ctx *ctx, const AttnArgs &a, int head_dim) {
    dim3 grid(a.nsplit, a.n_head / a.gc);
    if (head_dim == 64) launch_split<64>(a, grid, ctx->stream);
    else launch_split<128>(a, grid, ctx->stream);
    KH_HIP(hipGetLastError());
    if (a.nsplit > 1) {
        if (head_dim == 64)
            hipLaunchKernelGGL((attn_merge_kernel<64>), dim3(a.n_head), dim3(256), 0, ctx->stream, a);
        else
            hipLaunchKernelGGL((attn_merge_kernel<128>), dim3(a.n_head), dim3(256), 0, ctx->stream, a);
        KH_HIP(hipGetLastError());
    }
    return KH_OK;
}

}  // namespace

size_t attend_ws_bytes(int n_head, int n_kv_head, int head_dim, size_t max_positions) {
    (void)n_kv_head;
    const size_t ns = (max_positions + 15) / 16 * (size_t)n_head;  // the smallest split size bounds the count
    return 4 * (3 * ns + ns * head_dim) + 1024;
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
        const size_t ns = (size_t)a.nsplit * n_head;
        if ((rc = ensure(ctx, ctx->ws, 4 * (3 * ns + ns * head_dim) + 1024))) return rc;
        carve(a, ctx->ws.ptr, head_dim);
    }
    return run(ctx, a, head_dim);
}

int launch_attend_devlen(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const float *k,
                         const float *v, size_t kstride, size_t vstride, const int32_t *len_dev, int plus_one,
                         size_t max_positions, float *out, void *ws) {
    if (max_positions == 0) return fail(KH_EINVAL, "attend: no positions");
    AttnArgs a;
    int rc = setup(ctx, a, n_head, n_kv_head, head_dim, q, k, v, kstride, vstride, max_positions, out);
    if (rc) return rc;
    a.len_dev = len_dev;
    a.plus_one = plus_one;
    carve(a, ws, head_dim);
    return run(ctx, a, head_dim);
}

}  // namespace kh
