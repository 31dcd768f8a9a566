// GQA decode attention over a device-resident KV cache, split along the
// sequence.
//
// Reference: model::attend (crates/llm/src/model/mod.rs:769-819) with
// tensor::dot (tensor.rs:220-235) and softmax_inplace (tensor.rs:297-308).
// The reference walks every cached key once per query head of a group; here a
// workgroup owns one KV head (or a slice of its query heads) and a run of
// positions, and reads each key and value row once for the whole group -- the
// restructuring the reference's own notes ask for (docs/engine.md:783-791).
//
// Three launches, so that the weights are the reference's exactly, including
// its skip of weights under 1e-8 (mod.rs:807), which needs the global max and
// sum before any value is weighed:
//   1. scores: s[h][t] = dot(q_h, k_t) * (1/sqrt(hd)), kept in scratch (it is
//      n_head*L floats against 2*L*kv_dim of cache, and stays in L2/MALL);
//      per split the max and sum of exp(s - max); the last split of a head
//      group to finish folds those into the global max M and 1/S.
//   2. values: w = exp(s - M) * (1/S), zero under 1e-8, acc += w * v_t; one
//      partial output per split.
//   3. merge: the partials summed over splits in split order.
// Every sum has a fixed order, so results are deterministic run to run.
#include "common.hpp"

namespace kh {
namespace {

constexpr int MAXG = 8;     // query heads per workgroup
constexpr int MAXP = 256;   // positions per split

struct AttnArgs {
    const float *q;
    const float *k;
    const float *v;
    size_t kstride, vstride;   // floats between consecutive positions
    int n_head, group, gc;     // group = n_head / n_kv_head; gc = heads per workgroup
    int L, P, nsplit;
    float scale;
    float *scores;             // [n_head][L]
    float *smax, *ssum;        // [n_head][nsplit]
    float *gmax, *ginv;        // [n_head]
    float *part;               // [nsplit][n_head][hd]
    unsigned *cnt;             // [n_head / gc], zero between calls
    float *out;                // [n_head][hd]
};

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

template <int HD>
__global__ __launch_bounds__(256) void attn_scores(AttnArgs a) {
    constexpr int DPL = HD / 16;  // dims per lane; 16 lanes cover one row
    const int split = blockIdx.x, hg = blockIdx.y;
    const int h0 = hg * a.gc;                 // first query head of this workgroup
    const int kvh = h0 / a.group;             // its KV head
    const int G = a.gc;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = lane & 15, pg = tid >> 4;  // dim slice, position group (0..15)
    const int t0 = split * a.P;
    const int t1 = min(a.L, t0 + a.P);
    __shared__ float s_lds[MAXG][MAXP];
    __shared__ int s_last;

    float qr[MAXG][DPL];
#pragma unroll
    for (int h = 0; h < MAXG; h++)
#pragma unroll
        for (int d = 0; d < DPL; d++) qr[h][d] = h < G ? a.q[(size_t)(h0 + h) * HD + sub * DPL + d] : 0.0f;

    for (int base = t0; base < t1; base += 16) {
        const int t = base + pg;
        const bool ok = t < t1;
        float kv[DPL];
        const float *kr = a.k + (size_t)(ok ? t : t0) * a.kstride + (size_t)kvh * HD + sub * DPL;
#pragma unroll
        for (int d = 0; d < DPL; d += 4) {
            float4 f = ok ? *reinterpret_cast<const float4 *>(kr + d) : make_float4(0.f, 0.f, 0.f, 0.f);
            kv[d] = f.x;
            kv[d + 1] = f.y;
            kv[d + 2] = f.z;
            kv[d + 3] = f.w;
        }
        float part[MAXG];
#pragma unroll
        for (int h = 0; h < MAXG; h++) {
            float s = 0.0f;
#pragma unroll
            for (int d = 0; d < DPL; d++) s = fmaf(qr[h][d], kv[d], s);
            s += __shfl_xor(s, 8);
            s += __shfl_xor(s, 4);
            s += __shfl_xor(s, 2);
            s += __shfl_xor(s, 1);
            part[h] = s;
        }
#pragma unroll
        for (int h = 0; h < MAXG; h++) {
            if (ok && h < G && sub == h) {
                const float s = part[h] * a.scale;  // dot(q, k) * scale, mod.rs:802
                a.scores[(size_t)(h0 + h) * a.L + t] = s;
                s_lds[h][t - t0] = s;
            }
        }
    }
    __syncthreads();

    // per-split max and sum of exp(s - max) for each head
    const int n = t1 - t0;
    for (int h = wave; h < G; h += 4) {
        float m = -INFINITY;
        for (int i = lane; i < n; i += 64) m = fmaxf(m, s_lds[h][i]);
        m = wave_max(m);
        float s = 0.0f;
        for (int i = lane; i < n; i += 64) s += expf(s_lds[h][i] - m);
        s = wave_sum(s);
        if (lane == 0) {
            a.smax[(size_t)(h0 + h) * a.nsplit + split] = m;
            a.ssum[(size_t)(h0 + h) * a.nsplit + split] = s;
        }
    }

    // the last split of this head group to finish folds the statistics
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        unsigned prev = __hip_atomic_fetch_add(&a.cnt[hg], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == (unsigned)(a.nsplit - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int h = wave; h < G; h += 4) {
        const float *sm = a.smax + (size_t)(h0 + h) * a.nsplit;
        const float *ss = a.ssum + (size_t)(h0 + h) * a.nsplit;
        float m = -INFINITY;
        for (int j = lane; j < a.nsplit; j += 64)
            m = fmaxf(m, __hip_atomic_load(sm + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        m = wave_max(m);
        float s = 0.0f;
        for (int j = lane; j < a.nsplit; j += 64) {
            float lj = __hip_atomic_load(ss + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            float mj = __hip_atomic_load(sm + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s += lj * expf(mj - m);
        }
        s = wave_sum(s);
        if (lane == 0) {
            a.gmax[h0 + h] = m;
            a.ginv[h0 + h] = 1.0f / s;  // inv = 1 / sum, tensor.rs:304
        }
    }
    if (tid == 0) __hip_atomic_store(&a.cnt[hg], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int HD>
__global__ __launch_bounds__(256) void attn_values(AttnArgs a) {
    constexpr int DPL = HD / 16;
    const int split = blockIdx.x, hg = blockIdx.y;
    const int h0 = hg * a.gc;
    const int kvh = h0 / a.group;
    const int G = a.gc;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = lane & 15, pg = tid >> 4;
    const int t0 = split * a.P;
    const int t1 = min(a.L, t0 + a.P);
    __shared__ float w_lds[MAXG][MAXP];
    __shared__ float red[4][MAXG][HD];

    for (int idx = tid; idx < G * a.P; idx += 256) {
        const int h = idx / a.P, tt = idx % a.P, t = t0 + tt;
        if (t < t1) {
            const float s = a.scores[(size_t)(h0 + h) * a.L + t];
            float w = expf(s - a.gmax[h0 + h]);
            w = w * a.ginv[h0 + h];
            w_lds[h][tt] = w < 1e-8f ? 0.0f : w;  // skipped, mod.rs:807
        }
    }
    __syncthreads();

    float acc[MAXG][DPL];
#pragma unroll
    for (int h = 0; h < MAXG; h++)
#pragma unroll
        for (int d = 0; d < DPL; d++) acc[h][d] = 0.0f;

    for (int base = t0; base < t1; base += 16) {
        const int t = base + pg;
        if (t < t1) {
            const float *vr = a.v + (size_t)t * a.vstride + (size_t)kvh * HD + sub * DPL;
            float vv[DPL];
#pragma unroll
            for (int d = 0; d < DPL; d += 4) {
                float4 f = *reinterpret_cast<const float4 *>(vr + d);
                vv[d] = f.x;
                vv[d + 1] = f.y;
                vv[d + 2] = f.z;
                vv[d + 3] = f.w;
            }
#pragma unroll
            for (int h = 0; h < MAXG; h++) {
                if (h < G) {
                    const float w = w_lds[h][t - t0];
#pragma unroll
                    for (int d = 0; d < DPL; d++) acc[h][d] = fmaf(w, vv[d], acc[h][d]);
                }
            }
        }
    }
    // position groups within the wave (lanes 16 and 32 apart), then the waves
#pragma unroll
    for (int h = 0; h < MAXG; h++)
#pragma unroll
        for (int d = 0; d < DPL; d++) {
            float x = acc[h][d];
            x += __shfl_xor(x, 16);
            x += __shfl_xor(x, 32);
            acc[h][d] = x;
        }
    if (lane < 16) {
#pragma unroll
        for (int h = 0; h < MAXG; h++)
            if (h < G)
#pragma unroll
                for (int d = 0; d < DPL; d++) red[wave][h][sub * DPL + d] = acc[h][d];
    }
    __syncthreads();
    for (int idx = tid; idx < G * HD; idx += 256) {
        const int h = idx / HD, d = idx % HD;
        float s = red[0][h][d];
        s += red[1][h][d];
        s += red[2][h][d];
        s += red[3][h][d];
        a.part[((size_t)split * a.n_head + h0 + h) * HD + d] = s;
    }
}

// out[h][d] = sum over splits, in order, of part[split][h][d]
__global__ __launch_bounds__(256) void attn_merge(AttnArgs a, int hd) {
    const int h = blockIdx.x;
    const int slices = 256 / hd;
    const int d = threadIdx.x % hd, sl = threadIdx.x / hd;
    __shared__ float red[256];
    float s = 0.0f;
    if (sl < slices)
        for (int j = sl; j < a.nsplit; j += slices) s += a.part[((size_t)j * a.n_head + h) * hd + d];
    red[threadIdx.x] = s;
    __syncthreads();
    if (sl == 0) {
        float t = red[d];
        for (int k = 1; k < slices; k++) t += red[k * hd + d];
        a.out[(size_t)h * hd + d] = t;
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
    if (n_positions > (size_t)INT32_MAX) return fail(KH_EINVAL, "attend: too many positions");

    AttnArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.kstride = kstride;
    a.vstride = vstride;
    a.n_head = n_head;
    a.group = n_head / n_kv_head;
    int gc = 1;
    for (int c = 1; c <= MAXG; c++)
        if (a.group % c == 0) gc = c;
    a.gc = gc;
    const int n_hg = n_head / gc;
    a.L = (int)n_positions;
    // about two workgroups per CU in total, 16..256 positions each
    int target = (2 * (ctx->cu_count > 0 ? ctx->cu_count : 256)) / n_hg;
    if (target < 1) target = 1;
    int P = (int)((n_positions + target - 1) / target);
    P = (P + 15) / 16 * 16;
    if (P < 16) P = 16;
    if (P > MAXP) P = MAXP;
    a.P = P;
    a.nsplit = (int)((n_positions + P - 1) / P);
    a.scale = 1.0f / sqrtf((float)head_dim);  // mod.rs:777
    a.out = out;

    const size_t nscores = (size_t)n_head * n_positions;
    const size_t nstat = (size_t)n_head * a.nsplit;
    const size_t npart = (size_t)a.nsplit * n_head * head_dim;
    const size_t bytes = 4 * (nscores + 2 * nstat + 2 * (size_t)n_head + npart) + 256;
    int rc = ensure(ctx, ctx->ws, bytes);
    if (rc) return rc;
    float *base = static_cast<float *>(ctx->ws.ptr);
    a.scores = base;
    a.smax = a.scores + nscores;
    a.ssum = a.smax + nstat;
    a.gmax = a.ssum + nstat;
    a.ginv = a.gmax + n_head;
    a.part = a.ginv + n_head;
    if ((size_t)n_hg * sizeof(unsigned) > ctx->counters.bytes)
        return fail(KH_EINVAL, "attend: too many head groups for the counter block");
    a.cnt = static_cast<unsigned *>(ctx->counters.ptr);

    dim3 grid(a.nsplit, n_hg), block(256);
    if (head_dim == 64) {
        hipLaunchKernelGGL(attn_scores<64>, grid, block, 0, ctx->stream, a);
        hipLaunchKernelGGL(attn_values<64>, grid, block, 0, ctx->stream, a);
    } else {
        hipLaunchKernelGGL(attn_scores<128>, grid, block, 0, ctx->stream, a);
        hipLaunchKernelGGL(attn_values<128>, grid, block, 0, ctx->stream, a);
    }
    hipLaunchKernelGGL(attn_merge, dim3(n_head), block, 0, ctx->stream, a, head_dim);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

}  // namespace kh
