// GQA decode attention over a device-resident KV cache, split along the
// sequence, in one launch.
//
// Reference: model::attend (crates/llm/src/model/mod.rs:769-819) with
// tensor::dot (tensor.rs:220-235) and softmax_inplace (tensor.rs:297-308).
// The reference walks every cached key once per query head; here a workgroup
// owns one KV head's query heads (up to 8 of them) and a run of P positions,
// and reads each key and value row once for the whole group -- the
// restructuring the reference's notes ask for (docs/engine.md:783-791).
//
// Per workgroup (split j): all its K and V rows are loaded up front (16
// lanes per row, 16 rows per pass); scores s = dot(q, k) * scale; local max
// m_j, l_j = sum exp(s - m_j), acc_j = sum exp(s - m_j) v, and the smallest
// score.  Splits are merged in two levels, each by the last workgroup to
// arrive (an atomic counter per group, reset by that workgroup): chunks of
// 16 splits, then the chunks.  A merge of parts (m_i, l_i, acc_i) is
//   M = max m_i,  l = sum l_i exp(m_i - M),  acc = sum exp(m_i - M) acc_i,
// and the output is acc * (1/S) with S the final l.
//
// The reference skips weights w = exp(s - M) / S below 1e-8 (mod.rs:807).  A
// split whose smallest score could fall under that threshold
// (s < M + ln S + ln 1e-8, checked with a margin) has its positions scored
// again by the final merger, and each skipped term w * v is taken back out.
// Real scores never qualify (it takes a gap of about 18 + ln S), so the fast
// path is the whole cost; the slow path keeps the reference's weights exact
// when it does occur.  Every sum has a fixed order, so results are
// deterministic run to run.
#include "common.hpp"

namespace kh {
namespace {

constexpr unsigned RSRC_WORD3 = 0x00020000;
constexpr int CH = 16;  // splits per first-level merge

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
    int L, P, nsplit, nchunk;
    float scale;
    // per split, [nsplit][n_head]: local max, sum, smallest score; and acc
    float *pm, *pl, *pmin, *pacc;
    // per chunk of CH splits, [nchunk][n_head] and [nchunk][n_head][hd]
    float *cm, *cl, *cmin, *cacc;
    unsigned *cnt_top;        // [n_head / gc]
    unsigned *cnt_chunk;      // [n_head / gc][nchunk]
    float *out;               // [n_head][hd]
};

// The 16-lane row's scores of one position for the G heads: the same
// arithmetic in the main pass and in the skip correction.
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

// Merges parts [first, first + np) of the head group's G heads into
// dst (m, l, min, acc at index `slot`).  Run by a whole workgroup.
template <int GM, int HD>
__device__ void merge_parts(const float *pm, const float *pl, const float *pmin, const float *pacc, int first,
                            int np, int n_head, int h0, int G, float *dm, float *dl, float *dmin, float *dacc,
                            int slot, float (*s_w)[CH]) {
    const int tid = threadIdx.x;
    // per head: max, then the weights exp(m_i - M), sum and min
    if (tid < G) {
        const int h = tid;
        float m[CH], l[CH], mn[CH];
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const size_t o = (size_t)(first + (i < np ? i : 0)) * n_head + h0 + h;
            m[i] = i < np ? pm[o] : -INFINITY;
            l[i] = i < np ? pl[o] : 0.0f;
            mn[i] = i < np ? pmin[o] : INFINITY;
        }
        float M = -INFINITY, lo = INFINITY;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            M = fmaxf(M, m[i]);
            lo = fminf(lo, mn[i]);
        }
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const float w = i < np ? expf(m[i] - M) : 0.0f;
            s_w[h][i] = w;
            sum = fmaf(l[i], w, sum);
        }
        const size_t od = (size_t)slot * n_head + h0 + h;
        dm[od] = M;
        dl[od] = sum;
        dmin[od] = lo;
    }
    __syncthreads();
    for (int i = tid; i < G * HD; i += 256) {
        const int h = i / HD, d = i % HD;
        float c[CH];
#pragma unroll
        for (int k = 0; k < CH; k++)
            c[k] = k < np ? pacc[((size_t)(first + k) * n_head + h0 + h) * HD + d] : 0.0f;
        float x = 0.0f;
#pragma unroll
        for (int k = 0; k < CH; k++)
            if (k < np) x = fmaf(s_w[h][k], c[k], x);
        dacc[((size_t)slot * n_head + h0 + h) * HD + d] = x;
    }
}

template <int HD, int GM, int NP>  // NP: passes of 16 positions; P = 16 * NP
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
    constexpr int DPL = HD / 16;  // dims per lane
    constexpr int P = 16 * NP;
    const int split = blockIdx.x, hg = blockIdx.y;
    const int h0 = hg * a.gc, kvh = h0 / a.group, G = a.gc;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = lane & 15, pg = tid >> 4;  // dim slice, position within a pass
    const int t0 = split * P;
    const int n = min(a.L - t0, P);
    const rsrc_t K = rsrc(a.k, a.kbytes), V = rsrc(a.v, a.vbytes);

    __shared__ float s_p[GM][P];          // scores, then exp(s - m)
    __shared__ float s_red[4][GM][HD];    // per-wave partial acc; merge output
    __shared__ float s_w[GM][CH];
    __shared__ int s_flag;

    // every K and V row of the split in flight at once
    float kr[NP][DPL], vr[NP][DPL];
#pragma unroll
    for (int u = 0; u < NP; u++) {
        const int t = t0 + u * 16 + pg;
        const unsigned ko = (unsigned)(((size_t)t * a.kstride + (size_t)kvh * HD + sub * DPL) * 4);
        const unsigned vo = (unsigned)(((size_t)t * a.vstride + (size_t)kvh * HD + sub * DPL) * 4);
#pragma unroll
        for (int d = 0; d < DPL; d += 4) {
            float4 f = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(K, ko, d * 4, 0));
            kr[u][d] = f.x, kr[u][d + 1] = f.y, kr[u][d + 2] = f.z, kr[u][d + 3] = f.w;
            f = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(V, vo, d * 4, 0));
            vr[u][d] = f.x, vr[u][d + 1] = f.y, vr[u][d + 2] = f.z, vr[u][d + 3] = f.w;
        }
    }
    float qr[GM][DPL];
#pragma unroll
    for (int h = 0; h < GM; h++)
#pragma unroll
        for (int d = 0; d < DPL; d++) qr[h][d] = h < G ? a.q[(size_t)(h0 + h) * HD + sub * DPL + d] : 0.0f;

    // scores
#pragma unroll
    for (int u = 0; u < NP; u++) {
        float s[GM];
        score_row<GM, DPL>(qr, kr[u], a.scale, G, s);
        const int tt = u * 16 + pg;
#pragma unroll
        for (int h = 0; h < GM; h++)
            if (sub == h && h < G) s_p[h][tt] = tt < n ? s[h] : -INFINITY;
    }
    __syncthreads();

    // local softmax statistics; weights exp(s - m) in place
    for (int h = wave; h < G; h += 4) {
        float mx = -INFINITY, mn = INFINITY;
        for (int i = lane; i < n; i += 64) {
            mx = fmaxf(mx, s_p[h][i]);
            mn = fminf(mn, s_p[h][i]);
        }
        mx = wave_max(mx);
        mn = wave_min(mn);
        float l = 0.0f;
        for (int i = lane; i < P; i += 64) {
            const float e = i < n ? expf(s_p[h][i] - mx) : 0.0f;
            s_p[h][i] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            const size_t o = (size_t)split * a.n_head + h0 + h;
            a.pm[o] = mx;
            a.pl[o] = l;
            a.pmin[o] = mn;
        }
    }
    __syncthreads();

    // acc[h][:] = sum_t exp(s_t - m) v_t over this lane's positions
    float acc[GM][DPL];
#pragma unroll
    for (int h = 0; h < GM; h++)
#pragma unroll
        for (int d = 0; d < DPL; d++) acc[h][d] = 0.0f;
#pragma unroll
    for (int u = 0; u < NP; u++) {
        const int tt = u * 16 + pg;
#pragma unroll
        for (int h = 0; h < GM; h++) {
            if (h < G) {
                const float p = s_p[h][tt];
#pragma unroll
                for (int d = 0; d < DPL; d++) acc[h][d] = fmaf(p, vr[u][d], acc[h][d]);
            }
        }
    }
    // the wave's four rows (lanes 16 and 32 apart), then the four waves
#pragma unroll
    for (int h = 0; h < GM; h++)
#pragma unroll
        for (int d = 0; d < DPL; d++) {
            float x = acc[h][d];
            x += __shfl_xor(x, 16);
            x += __shfl_xor(x, 32);
            acc[h][d] = x;
        }
    if (lane < 16) {
#pragma unroll
        for (int h = 0; h < GM; h++)
            if (h < G)
#pragma unroll
                for (int d = 0; d < DPL; d++) s_red[wave][h][sub * DPL + d] = acc[h][d];
    }
    __syncthreads();
    for (int i = tid; i < G * HD; i += 256) {
        const int h = i / HD, d = i % HD;
        float x = s_red[0][h][d];
        x += s_red[1][h][d];
        x += s_red[2][h][d];
        x += s_red[3][h][d];
        a.pacc[((size_t)split * a.n_head + h0 + h) * HD + d] = x;
    }

    // ---- first level: the last split of a chunk merges the chunk -----------
    const int chunk = split / CH, cfirst = chunk * CH, cn = min(CH, a.nsplit - cfirst);
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        unsigned *c = &a.cnt_chunk[(size_t)hg * a.nchunk + chunk];
        const unsigned prev = __hip_atomic_fetch_add(c, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_flag = prev == (unsigned)(cn - 1);
        if (s_flag) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_flag) return;
    __threadfence();
    // a single chunk is the whole sequence: its merger is the final one
    const float *fm = a.pm, *fl = a.pl, *fmin = a.pmin, *facc = a.pacc;
    int nparts = a.nsplit;
    if (a.nchunk > 1) {
        merge_parts<GM, HD>(a.pm, a.pl, a.pmin, a.pacc, cfirst, cn, a.n_head, h0, G, a.cm, a.cl, a.cmin, a.cacc,
                            chunk, s_w);
        // ---- second level: the last chunk merges the chunks ----------------
        __threadfence();
        __syncthreads();
        if (tid == 0) {
            const unsigned prev =
                __hip_atomic_fetch_add(&a.cnt_top[hg], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            s_flag = prev == (unsigned)(a.nchunk - 1);
            if (s_flag) __hip_atomic_store(&a.cnt_top[hg], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!s_flag) return;
        __threadfence();
        fm = a.cm, fl = a.cl, fmin = a.cmin, facc = a.cacc;
        nparts = a.nchunk;
    }
    // the parts merged CH at a time, in order, into running (M, S, acc)
    __shared__ float s_M[GM], s_S[GM], s_min[GM], s_alpha[GM], s_inv[GM];
    if (tid < G) {
        s_M[tid] = -INFINITY;
        s_S[tid] = 0.0f;
        s_min[tid] = INFINITY;
    }
    for (int i = tid; i < G * HD; i += 256) s_red[0][i / HD][i % HD] = 0.0f;
    __syncthreads();
    for (int first = 0; first < nparts; first += CH) {
        const int np = min(CH, nparts - first);
        if (tid < G) {
            const int h = tid;
            float m[CH], l[CH], mn[CH];
#pragma unroll
            for (int i = 0; i < CH; i++) {
                const size_t o = (size_t)(first + (i < np ? i : 0)) * a.n_head + h0 + h;
                m[i] = i < np ? fm[o] : -INFINITY;
                l[i] = i < np ? fl[o] : 0.0f;
                mn[i] = i < np ? fmin[o] : INFINITY;
            }
            float M = s_M[h], lo = s_min[h];
#pragma unroll
            for (int i = 0; i < CH; i++) {
                M = fmaxf(M, m[i]);
                lo = fminf(lo, mn[i]);
            }
            const float alpha = s_M[h] == -INFINITY ? 0.0f : expf(s_M[h] - M);  // rescales the running sum
            float sum = s_S[h] * alpha;
#pragma unroll
            for (int i = 0; i < CH; i++) {
                const float w = i < np ? expf(m[i] - M) : 0.0f;
                s_w[h][i] = w;
                sum = fmaf(l[i], w, sum);
            }
            s_alpha[h] = alpha;
            s_M[h] = M;
            s_S[h] = sum;
            s_min[h] = lo;
        }
        __syncthreads();
        for (int i = tid; i < G * HD; i += 256) {
            const int h = i / HD, d = i % HD;
            float c[CH];
#pragma unroll
            for (int k = 0; k < CH; k++)
                c[k] = k < np ? facc[((size_t)(first + k) * a.n_head + h0 + h) * HD + d] : 0.0f;
            float x = s_red[0][h][d] * s_alpha[h];
#pragma unroll
            for (int k = 0; k < CH; k++)
                if (k < np) x = fmaf(s_w[h][k], c[k], x);
            s_red[0][h][d] = x;
        }
        __syncthreads();
    }
    if (tid < G) s_inv[tid] = 1.0f / s_S[tid];  // inv = 1 / sum, tensor.rs:304
    __syncthreads();
    for (int i = tid; i < G * HD; i += 256) s_red[0][i / HD][i % HD] *= s_inv[i / HD];

    // ---- skip correction: w = exp(s - M) * (1/S) < 1e-8 ---------------------
    // possible only where a score is below M + ln S + ln 1e-8 (with a margin)
    if (tid == 0) {
        int need = 0;
        for (int h = 0; h < G; h++) need |= s_min[h] < s_M[h] + logf(s_S[h]) - 18.420681f + 1.0f;
        s_flag = need;
    }
    __syncthreads();
    if (s_flag) {
        for (int j = 0; j < a.nsplit; j++) {
            if (tid == 0) {
                int need = 0;
                for (int h = 0; h < G; h++)
                    need |= a.pmin[(size_t)j * a.n_head + h0 + h] < s_M[h] + logf(s_S[h]) - 18.420681f + 1.0f;
                s_flag = need;
            }
            __syncthreads();
            if (!s_flag) continue;
            const int tj = j * P, nj = min(a.L - tj, P);
            for (int base = 0; base < nj; base += 16) {
                const int t = tj + base + pg;
                const bool ok = base + pg < nj;
                float kv[DPL], vv[DPL];
                const unsigned ko = (unsigned)(((size_t)(ok ? t : tj) * a.kstride + (size_t)kvh * HD + sub * DPL) * 4);
                const unsigned vo = (unsigned)(((size_t)(ok ? t : tj) * a.vstride + (size_t)kvh * HD + sub * DPL) * 4);
#pragma unroll
                for (int d = 0; d < DPL; d += 4) {
                    float4 f = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(K, ko, d * 4, 0));
                    kv[d] = f.x, kv[d + 1] = f.y, kv[d + 2] = f.z, kv[d + 3] = f.w;
                    f = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(V, vo, d * 4, 0));
                    vv[d] = f.x, vv[d + 1] = f.y, vv[d + 2] = f.z, vv[d + 3] = f.w;
                }
                float s[GM];
                score_row<GM, DPL>(qr, kv, a.scale, G, s);
                // positions taken out one at a time, in order
                for (int r = 0; r < 16; r++) {
                    if (pg == r && ok) {
#pragma unroll
                        for (int h = 0; h < GM; h++) {
                            if (h < G) {
                                float w = expf(s[h] - s_M[h]);
                                w = w * s_inv[h];
                                if (w < 1e-8f) {
#pragma unroll
                                    for (int d = 0; d < DPL; d++) s_red[0][h][sub * DPL + d] -= w * vv[d];
                                }
                            }
                        }
                    }
                    __syncthreads();
                }
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < G * HD; i += 256) {
        const int h = i / HD, d = i % HD;
        a.out[(size_t)(h0 + h) * HD + d] = s_red[0][h][d];
    }
}

template <int HD, int GM>
void launch_g(const AttnArgs &a, dim3 grid, hipStream_t stream) {
    switch (a.P / 16) {
        case 1: hipLaunchKernelGGL((attn_kernel<HD, GM, 1>), grid, dim3(256), 0, stream, a); break;
        case 2: hipLaunchKernelGGL((attn_kernel<HD, GM, 2>), grid, dim3(256), 0, stream, a); break;
        case 4: hipLaunchKernelGGL((attn_kernel<HD, GM, 4>), grid, dim3(256), 0, stream, a); break;
        case 8: hipLaunchKernelGGL((attn_kernel<HD, GM, 8>), grid, dim3(256), 0, stream, a); break;
        default: hipLaunchKernelGGL((attn_kernel<HD, GM, (HD == 64 ? 16 : 8)>), grid, dim3(256), 0, stream, a); break;
    }
}

}  // namespace

int launch_attend(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const float *k,
                  const float *v, size_t kstride, size_t vstride, size_t n_positions, float *out) {
    if (n_kv_head <= 0 || n_head <= 0 || n_head % n_kv_head != 0)
        return fail(KH_EINVAL, "attend: n_head must be a positive multiple of n_kv_head");
    if (head_dim != 64 && head_dim != 128)
        return fail(KH_DECLINED, "attend: head_dim other than 64 or 128 runs on the CPU");
    if (n_positions == 0) return launch_fill(ctx, out, (size_t)n_head * head_dim, 0.0f);
    if ((n_positions * kstride + 4096) * 4 >= 0xffffffffull || (n_positions * vstride + 4096) * 4 >= 0xffffffffull)
        return fail(KH_DECLINED, "attend: caches of 4 GiB or more per layer are not addressed here");

    AttnArgs a{};
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
    // positions per split: a power-of-two count of 16-row passes, growing
    // until the launch is about one workgroup per CU (at most 256 rows for
    // hd 64, 128 for hd 128)
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const int pmax = head_dim == 64 ? 256 : 128;
    int P = 16;
    while (P < pmax && (long long)((n_positions + P - 1) / P) * n_hg > cu) P *= 2;
    a.P = P;
    a.nsplit = (int)((n_positions + P - 1) / P);
    a.nchunk = (a.nsplit + CH - 1) / CH;
    a.scale = 1.0f / sqrtf((float)head_dim);  // mod.rs:777
    a.out = out;

    const size_t ns = (size_t)a.nsplit * n_head, nc = (size_t)a.nchunk * n_head;
    const size_t bytes = 4 * (3 * ns + ns * head_dim + 3 * nc + nc * head_dim) + 1024;
    int rc = ensure(ctx, ctx->ws, bytes);
    if (rc) return rc;
    float *p = static_cast<float *>(ctx->ws.ptr);
    a.pm = p, p += ns;
    a.pl = p, p += ns;
    a.pmin = p, p += ns;
    a.pacc = p, p += ns * head_dim;
    a.cm = p, p += nc;
    a.cl = p, p += nc;
    a.cmin = p, p += nc;
    a.cacc = p;
    const size_t ncounters = (size_t)n_hg * (1 + a.nchunk);
    if (ncounters * sizeof(unsigned) > ctx->counters.bytes)
        return fail(KH_DECLINED, "attend: sequence too long for the counter block");
    a.cnt_top = static_cast<unsigned *>(ctx->counters.ptr);
    a.cnt_chunk = a.cnt_top + n_hg;

    dim3 grid(a.nsplit, n_hg);
    if (head_dim == 64) {
        if (gc <= 4) launch_g<64, 4>(a, grid, ctx->stream);
        else launch_g<64, 8>(a, grid, ctx->stream);
    } else {
        if (gc <= 4) launch_g<128, 4>(a, grid, ctx->stream);
        else launch_g<128, 8>(a, grid, ctx->stream);
    }
    KH_HIP(hipGetLastError());
    return KH_OK;
}

}  // namespace kh
