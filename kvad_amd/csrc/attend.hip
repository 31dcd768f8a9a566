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

template <int HD, int GM, int NP>  // NP: passes of 16 positions; P = 16 * NP
__global__ __launch_bounds__(256) void attn_split_kernel(AttnArgs a) {
    constexpr int DPL = HD / 16;  // dims per lane
    constexpr int P = 16 * NP;
    const int split = blockIdx.x, hg = blockIdx.y;
    const int h0 = hg * a.gc, kvh = h0 / a.group, G = a.gc;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = lane & 15, pg = tid >> 4;  // dim slice, position within a pass
    const int t0 = split * P;
    const int n = min(a.L - t0, P);
    const bool whole = a.nsplit == 1;
    const rsrc_t K = rsrc(a.k, a.kbytes), V = rsrc(a.v, a.vbytes);

    __shared__ float s_p[GM][P];          // scores, then exp(s - m) (or final weights)
    __shared__ float s_red[4][GM][HD];    // per-wave partial acc

    // every K and V row of the split in flight at once
    float kr[NP][DPL], vr[NP][DPL];
#pragma unroll
    for (int u = 0; u < NP; u++) {
        const size_t t = (size_t)(t0 + u * 16 + pg);
        load_row<DPL>(K, (unsigned)((t * a.kstride + (size_t)kvh * HD + sub * DPL) * 4), kr[u]);
        load_row<DPL>(V, (unsigned)((t * a.vstride + (size_t)kvh * HD + sub * DPL) * 4), vr[u]);
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

    // local softmax statistics (softmax_inplace, tensor.rs:297-308); exp(s - m)
    // in place, or, for a whole sequence, the final weights
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
        if (whole) {
            const float inv = 1.0f / l;
            for (int i = lane; i < P; i += 64) {
                const float w = s_p[h][i] * inv;
                s_p[h][i] = w < 1e-8f ? 0.0f : w;  // mod.rs:807
            }
        } else if (lane == 0) {
            const size_t o = (size_t)split * a.n_head + h0 + h;
            a.pm[o] = mx;
            a.pl[o] = l;
            a.pmin[o] = mn;
        }
    }
    __syncthreads();

    // acc[h][:] = sum_t p_t v_t over this lane's positions
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
    float *dst = whole ? a.out + (size_t)h0 * HD : a.pacc + ((size_t)split * a.n_head + h0) * HD;
    for (int i = tid; i < G * HD; i += 256) {
        const int h = i / HD, d = i % HD;
        float x = s_red[0][h][d];
        x += s_red[1][h][d];
        x += s_red[2][h][d];
        x += s_red[3][h][d];
        dst[(size_t)h * HD + d] = x;
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

template <int HD>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnArgs a) {
    constexpr int DPL = HD / 16, NG = 256 / HD;  // dim groups of the acc merge
    const int h = blockIdx.x, tid = threadIdx.x;
    const int ns = a.nsplit, n_head = a.n_head;
    __shared__ float s_red[256];
    __shared__ float s_acc[NG][HD];
    __shared__ float s_fix[16][HD];
    __shared__ int s_need;

    // M and the smallest score over the splits
    float mx = -INFINITY, lo = INFINITY;
    for (int i = tid; i < ns; i += 256) {
        mx = fmaxf(mx, a.pm[(size_t)i * n_head + h]);
        lo = fminf(lo, a.pmin[(size_t)i * n_head + h]);
    }
    const float M = block_reduce(mx, s_red, [](float x, float y) { return fmaxf(x, y); });
    lo = block_reduce(lo, s_red, [](float x, float y) { return fminf(x, y); });

    // S = sum l_j exp(m_j - M)
    float s = 0.0f;
    for (int i = tid; i < ns; i += 256) {
        const size_t o = (size_t)i * n_head + h;
        s = fmaf(a.pl[o], expf(a.pm[o] - M), s);
    }
    const float S = block_reduce(s, s_red, [](float x, float y) { return x + y; });
    const float inv = 1.0f / S;  // inv = 1 / sum, tensor.rs:304

    // acc[d] = sum_j exp(m_j - M) acc_j[d]
    {
        const int g = tid / HD, d = tid % HD;
        float x = 0.0f;
        for (int i = g; i < ns; i += NG) {
            const size_t o = (size_t)i * n_head + h;
            x = fmaf(expf(a.pm[o] - M), a.pacc[o * HD + d], x);
        }
        s_acc[g][d] = x;
    }
    __syncthreads();

    // ---- skip correction: w = exp(s - M) * (1/S) < 1e-8 ---------------------
    // possible only where a score is below M + ln S + ln 1e-8 (with a margin)
    const float thr = M + logf(S) - 18.420681f + 1.0f;
    if (lo < thr) {
        const int group16 = tid >> 4, sub = tid & 15, kvh = h / a.group;
        const rsrc_t K = rsrc(a.k, a.kbytes), V = rsrc(a.v, a.vbytes);
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
            const int tj = j * a.P, nj = min(a.L - tj, a.P);
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
        for (int g = 1; g < NG; g++) x += s_acc[g][tid];
        x = x * inv;
        if (lo < thr) x -= s_fix[0][tid];
        a.out[(size_t)h * HD + tid] = x;
    }
}

template <int HD, int GM>
void launch_split(const AttnArgs &a, dim3 grid, hipStream_t stream) {
    switch (a.P / 16) {
        case 1: hipLaunchKernelGGL((attn_split_kernel<HD, GM, 1>), grid, dim3(256), 0, stream, a); break;
        case 2: hipLaunchKernelGGL((attn_split_kernel<HD, GM, 2>), grid, dim3(256), 0, stream, a); break;
        case 4: hipLaunchKernelGGL((attn_split_kernel<HD, GM, 4>), grid, dim3(256), 0, stream, a); break;
        case 8: hipLaunchKernelGGL((attn_split_kernel<HD, GM, 8>), grid, dim3(256), 0, stream, a); break;
        default: hipLaunchKernelGGL((attn_split_kernel<HD, GM, (HD == 64 ? 16 : 8)>), grid, dim3(256), 0, stream, a); break;
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
    // 32-bit buffer offsets, including a split's overhang past the last row
    if ((n_positions + 256) * kstride * 4 >= 0xffffffffull || (n_positions + 256) * vstride * 4 >= 0xffffffffull)
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
    a.scale = 1.0f / sqrtf((float)head_dim);  // mod.rs:777
    a.out = out;

    if (a.nsplit > 1) {
        const size_t ns = (size_t)a.nsplit * n_head;
        const size_t bytes = 4 * (3 * ns + ns * head_dim) + 1024;
        int rc = ensure(ctx, ctx->ws, bytes);
        if (rc) return rc;
        float *p = static_cast<float *>(ctx->ws.ptr);
        a.pm = p, p += ns;
        a.pl = p, p += ns;
        a.pmin = p, p += ns;
        a.pacc = p;
    }

    dim3 grid(a.nsplit, n_hg);
    if (head_dim == 64) {
        if (gc <= 4) launch_split<64, 4>(a, grid, ctx->stream);
        else launch_split<64, 8>(a, grid, ctx->stream);
    } else {
        if (gc <= 4) launch_split<128, 4>(a, grid, ctx->stream);
        else launch_split<128, 8>(a, grid, ctx->stream);
    }
    KH_HIP(hipGetLastError());
    if (a.nsplit > 1) {
        if (head_dim == 64)
            hipLaunchKernelGGL((attn_merge_kernel<64>), dim3(n_head), dim3(256), 0, ctx->stream, a);
        else
            hipLaunchKernelGGL((attn_merge_kernel<128>), dim3(n_head), dim3(256), 0, ctx->stream, a);
        KH_HIP(hipGetLastError());
    }
    return KH_OK;
}

}  // namespace kh
