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

// Split kernel.  Lanes form 16-lane rows (16 per workgroup); row r takes
// positions r, r + 16, ... of the split, lane `sub` of a row dims
// [sub*DPL, sub*DPL + DPL).  Each wave reduces its four rows with lane swaps
// against the wave's own maximum, and the four waves meet once in LDS.
template <int HD, int G, int NP>  // G heads per workgroup; P = 16 * NP positions
__global__ __launch_bounds__(256) void attn_split_kernel(AttnArgs a) {
    constexpr int DPL = HD / 16;  // dims per lane
    constexpr int P = 16 * NP;
    const int split = blockIdx.x, hg = blockIdx.y;
    const int h0 = hg * G, kvh = h0 / a.group;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = lane & 15, row = tid >> 4;
    const int L = a.len_dev ? min(*a.len_dev + a.plus_one, a.L) : a.L;
    const int nsplit = (L + P - 1) / P;
    if (split >= nsplit) return;
    const int t0 = split * P;
    const int n = min(L - t0, P);
    const bool whole = nsplit == 1;
    const rsrc_t K = rsrc(a.k, (size_t)L * a.kstride * 4), V = rsrc(a.v, (size_t)L * a.vstride * 4);

    __shared__ float s_acc[4][G][HD];  // per-wave totals
    __shared__ float s_st[3][4][G];    // per-wave max, sum, smallest score

    // every K and V row of the split in flight at once
    float kr[NP][DPL], vr[NP][DPL];
#pragma unroll
    for (int u = 0; u < NP; u++) {
        const size_t t = (size_t)(t0 + u * 16 + row);
        load_row<DPL>(K, (unsigned)((t * a.kstride + (size_t)kvh * HD + sub * DPL) * 4), kr[u]);
        load_row<DPL>(V, (unsigned)((t * a.vstride + (size_t)kvh * HD + sub * DPL) * 4), vr[u]);
    }
    float qr[G][DPL];
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int d = 0; d < DPL; d += 4) {
            const float4 f = *reinterpret_cast<const float4 *>(a.q + (size_t)(h0 + h) * HD + sub * DPL + d);
            qr[h][d] = f.x, qr[h][d + 1] = f.y, qr[h][d + 2] = f.z, qr[h][d + 3] = f.w;
        }

    // scores (the same in all 16 lanes of a row), the row's extremes
    float s[NP][G], mx[G], mn[G];
#pragma unroll
    for (int h = 0; h < G; h++) mx[h] = -INFINITY, mn[h] = INFINITY;
#pragma unroll
    for (int u = 0; u < NP; u++) {
        score_row<G, DPL>(qr, kr[u], a.scale, G, s[u]);
        const bool ok = u * 16 + row < n;
#pragma unroll
        for (int h = 0; h < G; h++) {
            s[u][h] = ok ? s[u][h] : -INFINITY;
            mx[h] = fmaxf(mx[h], s[u][h]);
            mn[h] = ok ? fminf(mn[h], s[u][h]) : mn[h];
        }
    }
#pragma unroll
    for (int h = 0; h < G; h++) {
        mx[h] = rows_max(mx[h]);
        mn[h] = rows_min(mn[h]);
    }

    // exp(s - m) against the wave's max; the wave's sum and weighted values
    float l[G], acc[G][DPL];
#pragma unroll
    for (int h = 0; h < G; h++) {
        l[h] = 0.0f;
#pragma unroll
        for (int d = 0; d < DPL; d++) acc[h][d] = 0.0f;
    }
#pragma unroll
    for (int u = 0; u < NP; u++)
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float e = s[u][h] == -INFINITY ? 0.0f : expf(s[u][h] - mx[h]);
            l[h] += e;
#pragma unroll
            for (int d = 0; d < DPL; d++) acc[h][d] = fmaf(e, vr[u][d], acc[h][d]);
        }
#pragma unroll
    for (int h = 0; h < G; h++) {
        l[h] = rows_sum(l[h]);
#pragma unroll
        for (int d = 0; d < DPL; d++) acc[h][d] = rows_sum(acc[h][d]);
    }
    if (lane < 16) {
#pragma unroll
        for (int h = 0; h < G; h++)
#pragma unroll
            for (int d = 0; d < DPL; d++) s_acc[wave][h][sub * DPL + d] = acc[h][d];
    }
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < G; h++) {
            s_st[0][wave][h] = mx[h];
            s_st[1][wave][h] = l[h];
            s_st[2][wave][h] = mn[h];
        }
    }
    __syncthreads();

    if (!whole) {
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
            float L = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float c = s_st[0][w][h] == -INFINITY ? 0.0f : expf(s_st[0][w][h] - M);
                L = fmaf(c, s_st[1][w][h], L);
            }
            const size_t o = (size_t)split * a.n_head + h0 + h;
            a.pm[o] = M;
            a.pl[o] = L;
            a.pmin[o] = fminf(fminf(s_st[2][0][h], s_st[2][1][h]), fminf(s_st[2][2][h], s_st[2][3][h]));
        }
        return;
    }

    // One split is the whole sequence: the reference's own weights
    // w = exp(s - M) * (1/S), S = sum exp(s - M), dropping w < 1e-8
    // (softmax_inplace, tensor.rs:297-308; mod.rs:805-812).
    float M[G];
#pragma unroll
    for (int h = 0; h < G; h++)
        M[h] = fmaxf(fmaxf(s_st[0][0][h], s_st[0][1][h]), fmaxf(s_st[0][2][h], s_st[0][3][h]));
    float e[NP][G];
#pragma unroll
    for (int h = 0; h < G; h++) l[h] = 0.0f;
#pragma unroll
    for (int u = 0; u < NP; u++)
#pragma unroll
        for (int h = 0; h < G; h++) {
            e[u][h] = s[u][h] == -INFINITY ? 0.0f : expf(s[u][h] - M[h]);
            l[h] += e[u][h];
        }
#pragma unroll
    for (int h = 0; h < G; h++) l[h] = rows_sum(l[h]);
    __syncthreads();  // everyone has read s_st
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < G; h++) s_st[1][wave][h] = l[h];
    }
    __syncthreads();
    float inv[G];
#pragma unroll
    for (int h = 0; h < G; h++) inv[h] = 1.0f / (((s_st[1][0][h] + s_st[1][1][h]) + s_st[1][2][h]) + s_st[1][3][h]);
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int d = 0; d < DPL; d++) acc[h][d] = 0.0f;
#pragma unroll
    for (int u = 0; u < NP; u++)
#pragma unroll
        for (int h = 0; h < G; h++) {
            float w = e[u][h] * inv[h];
            w = w < 1e-8f ? 0.0f : w;
#pragma unroll
            for (int d = 0; d < DPL; d++) acc[h][d] = fmaf(w, vr[u][d], acc[h][d]);
        }
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int d = 0; d < DPL; d++) acc[h][d] = rows_sum(acc[h][d]);
    if (lane < 16) {
#pragma unroll
        for (int h = 0; h < G; h++)
#pragma unroll
            for (int d = 0; d < DPL; d++) s_acc[wave][h][sub * DPL + d] = acc[h][d];
    }
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

// P ladders: 16, 64, 128 positions for hd 64; 16, 32, 64 for hd 128.
template <int HD, int G>
void launch_split_g(const AttnArgs &a, dim3 grid, hipStream_t stream) {
    const int np = a.P / 16;
    if (np == 1) {
        hipLaunchKernelGGL((attn_split_kernel<HD, G, 1>), grid, dim3(256), 0, stream, a);
    } else if constexpr (HD == 64) {
        if (np == 4) hipLaunchKernelGGL((attn_split_kernel<64, G, 4>), grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((attn_split_kernel<64, G, 8>), grid, dim3(256), 0, stream, a);
    } else {
        if (np == 2) hipLaunchKernelGGL((attn_split_kernel<128, G, 2>), grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((attn_split_kernel<128, G, 4>), grid, dim3(256), 0, stream, a);
    }
}

template <int HD>
void launch_split(const AttnArgs &a, dim3 grid, hipStream_t stream) {
    switch (a.gc) {
        case 1: launch_split_g<HD, 1>(a, grid, stream); break;
        case 2: launch_split_g<HD, 2>(a, grid, stream); break;
        case 3: launch_split_g<HD, 3>(a, grid, stream); break;
        case 4: launch_split_g<HD, 4>(a, grid, stream); break;
        case 5: launch_split_g<HD, 5>(a, grid, stream); break;
        case 6: launch_split_g<HD, 6>(a, grid, stream); break;
        case 7: launch_split_g<HD, 7>(a, grid, stream); break;
        default: launch_split_g<HD, 8>(a, grid, stream); break;
    }
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
    int gc = 1;
    for (int c = 1; c <= 8; c++)
        if (a.group % c == 0) gc = c;
    a.gc = gc;
    const int n_hg = n_head / gc;
    a.L = (int)n_positions;
    // positions per split, from a short ladder: 16 rows, or the middle rung
    // when that would give more than about four workgroups per CU, or the
    // top rung when the merge's split limit needs it
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const int ladder[3] = {16, head_dim == 64 ? 64 : 32, head_dim == 64 ? 128 : 64};
    int step = 0;
    while (step < 1 && (long long)((n_positions + ladder[step] - 1) / ladder[step]) * n_hg > 4 * cu) step++;
    while (step < 2 && (n_positions + ladder[step] - 1) / ladder[step] > (size_t)MAX_SPLITS) step++;
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
