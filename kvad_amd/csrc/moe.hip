// A mixture-of-experts layer on the device: Moe::run (crates/llm/src/model/
// ffn.rs:615-708) with Router::route (ffn.rs:256-349), mix (ffn.rs:744-806),
// decode_together (ffn.rs:820-842) and SharedExpert::run (ffn.rs:437-451).
//
// Decode (one token) is three GEMV launches and the combine, with no host
// round trip: (1) one GEMV launch for the router and the shared expert's
// gate and up, which read the same input, (2) in whose router workgroup one
// wave routes the logits and writes the chosen experts in expert order (a
// launch of its own where the GEMV has no routing build for the shape);
// (3) one GEMV launch for every chosen expert's gate and up, each job
// reading its weight through a device table indexed by the router's pick; (4) one GEMV launch for every down projection, the shared expert's
// included, each staging swiglu(gate, up) as its input; then the combine,
// which adds the weighted expert outputs to the shared expert's in expert
// order -- the order mix() adds them, so the sum rounds as the reference's.
//
// Prefill groups the tokens by expert (expert order, then token order, as
// by_expert is filled, ffn.rs:627-640), runs every expert's gate and up as
// one grouped int8 GEMM launch over tiles of its rows (the two weight tables
// paired) and every down as another, and combines per token in expert order
// after the shared expert (which runs on every token, its gate and up paired
// the same way).  The input rows are quantised once, for the router too.
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.hpp"
#include "route.hpp"

namespace kh {
namespace {


// Router::route for one token per wave (route.hpp).
__global__ __launch_bounds__(64) void route_kernel(RouteArgs r) {
    route_one(r, blockIdx.x, r.logits + (size_t)blockIdx.x * r.n);
}

typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t rsrc(const void *p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)(bytes > 0xffffffffu ? 0xffffffffu : bytes), 0x00020000);
}

// A batch's routes with each token's logits made in its own workgroup (q8
// routers), in place of the router GEMM, its split-K reduce and route_kernel:
// token blockIdx.x's quantised row (the QActBatch::new codes and scales every
// expert reads) against every router row -- per 32-block the exact i32 dot
// scaled by ws * xs (qrow pass 2, quant.rs:443-451), the row's blocks summed
// in each lane (blocks lane, lane + 64, ...) and then over the wave by a
// fixed butterfly -- into LDS and `logits`, then route_one over them.  Each
// wave takes rows wave * ER + i of every group of 4 * ER rows, all their
// loads in flight together.  Rows and blocks past the ends read zeros.
template <int NB>
__global__ __launch_bounds__(256) void route_rows_kernel(RouteArgs r, float *logits, const int8_t *xq, const float *xs,
                                                         const int8_t *wq, const float *wsc, int cols) {
    constexpr int ER = 16 / NB;  // rows a wave has in flight
    __shared__ float s_lg[MAX_EXPERTS];
    const int tok = blockIdx.x, lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = cols / BLOCK, n = r.n;
    const rsrc_t X = rsrc(xq + (size_t)tok * cols, (size_t)cols);
    const rsrc_t XS = rsrc(xs + (size_t)tok * nb, (size_t)nb * 4);
    const rsrc_t W = rsrc(wq, (size_t)n * cols);
    const rsrc_t WS = rsrc(wsc, (size_t)n * nb * 4);
    auto ld16 = [](const rsrc_t &q, unsigned off) {
        return __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(q, off, 0, 0));
    };
    auto ldf = [](const rsrc_t &q, unsigned off) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(q, off, 0, 0));
    };
    constexpr unsigned OOB = 0xffffffffu;
    int4 a[NB][2];
    float as[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const int b = lane + 64 * j;
        const unsigned o = b < nb ? (unsigned)b * BLOCK : OOB;
        a[j][0] = ld16(X, o), a[j][1] = ld16(X, o == OOB ? OOB : o + 16);
        as[j] = ldf(XS, b < nb ? (unsigned)b * 4 : OOB);
    }
    for (int e0 = wave * ER; e0 < n; e0 += 4 * ER) {
        int4 w[ER][NB][2];
        float s[ER][NB];
#pragma unroll
        for (int i = 0; i < ER; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) {
                const int e = e0 + i, b = lane + 64 * j;
                const bool ok = e < n && b < nb;
                const unsigned o = ok ? (unsigned)e * (unsigned)cols + (unsigned)b * BLOCK : OOB;
                w[i][j][0] = ld16(W, o), w[i][j][1] = ld16(W, ok ? o + 16 : OOB);
                s[i][j] = ldf(WS, ok ? ((unsigned)e * (unsigned)nb + (unsigned)b) * 4 : OOB);
            }
        __builtin_amdgcn_sched_barrier(0);  // every row's loads in flight before the first dot
        float acc[ER];
#pragma unroll
        for (int i = 0; i < ER; i++) {
            acc[i] = 0.0f;
#pragma unroll
            for (int j = 0; j < NB; j++) {
                int d = __builtin_amdgcn_sdot4(w[i][j][0].x, a[j][0].x, 0, false);
                d = __builtin_amdgcn_sdot4(w[i][j][0].y, a[j][0].y, d, false);
                d = __builtin_amdgcn_sdot4(w[i][j][0].z, a[j][0].z, d, false);
                d = __builtin_amdgcn_sdot4(w[i][j][0].w, a[j][0].w, d, false);
                d = __builtin_amdgcn_sdot4(w[i][j][1].x, a[j][1].x, d, false);
                d = __builtin_amdgcn_sdot4(w[i][j][1].y, a[j][1].y, d, false);
                d = __builtin_amdgcn_sdot4(w[i][j][1].z, a[j][1].z, d, false);
                d = __builtin_amdgcn_sdot4(w[i][j][1].w, a[j][1].w, d, false);
                const float sc = s[i][j] * as[j];
                acc[i] += sc * (float)d;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
#pragma unroll
            for (int i = 0; i < ER; i++) acc[i] += __shfl_xor(acc[i], o);
        if (lane < ER && e0 + lane < n) {
            float v = acc[0];
#pragma unroll
            for (int i = 1; i < ER; i++) v = lane == i ? acc[i] : v;
            s_lg[e0 + lane] = v;
            logits[(size_t)tok * n + e0 + lane] = v;
        }
    }
    __syncthreads();
    if (wave == 0) route_one(r, tok, s_lg);
}

// by_expert (ffn.rs:627-640): the picks' rows grouped by expert, experts in
// order.  Within an expert the rows are placed by LDS atomics, in no fixed
// order: no output depends on it (each row's products and its mix are its
// own; pos records where every pick went).  One workgroup of 1024 threads:
// (1) the picks per expert, (2) exclusive prefixes over experts of rows and
// of tile_m-row tiles, each expert writing its own tiles, (3) each pick's
// row.  For the mix, each token's rows and weights are also written in
// expert order (pos, wpos), the order of ffn.rs:775-805.
constexpr int GROUP_THREADS = 1024;
constexpr int GROUP_PICKS = 8192;  // picks (tokens x top_k) staged in LDS when they fit

// Exclusive prefix of v over the workgroup's threads in thread order; `total`
// gets the sum.  Every thread calls it.
__device__ int group_scan(int v, int *s_wave, int &total) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    constexpr int NW = GROUP_THREADS / 64;
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    if (lane == 63) s_wave[w] = x;
    __syncthreads();
    if (tid < 64) {
        int y = tid < NW ? s_wave[tid] : 0;
#pragma unroll
        for (int d = 1; d < NW; d <<= 1) {
            const int z = __shfl_up(y, d, 64);
            if (lane >= d) y += z;
        }
        if (tid < NW) s_wave[tid] = y;
    }
    __syncthreads();
    total = s_wave[NW - 1];
    const int r = (w ? s_wave[w - 1] : 0) + x - v;
    __syncthreads();  // s_wave free again
    return r;
}

__global__ __launch_bounds__(GROUP_THREADS) void group_kernel(const int32_t *experts, const float *weights,
                                                             const int32_t *count, int m, int top_k, int n_exp,
                                                             int tile_m, int32_t *row_token, float *row_weight,
                                                             int32_t *pos, float *wpos, int32_t *tiles) {
    __shared__ int s_cnt[MAX_EXPERTS];  // picks per expert, then its next free row
    __shared__ int s_wave[GROUP_THREADS / 64];
    __shared__ int s_exp[GROUP_PICKS], s_count[GROUP_PICKS];
    const int tid = threadIdx.x;
    const bool staged = m * top_k <= GROUP_PICKS;
    for (int x = tid; x < n_exp; x += GROUP_THREADS) s_cnt[x] = 0;
    if (staged) {
        for (int i = tid; i < m * top_k; i += GROUP_THREADS) s_exp[i] = experts[i];
        for (int t = tid; t < m; t += GROUP_THREADS) s_count[t] = count[t];
    }
    __syncthreads();
    const int *E = staged ? s_exp : experts, *C = staged ? s_count : count;
    for (int i = tid; i < m * top_k; i += GROUP_THREADS) {
        const int t = i / top_k, k = i % top_k;
        if (k < C[t]) atomicAdd(&s_cnt[E[i]], 1);
    }
    __syncthreads();
    // n_exp <= MAX_EXPERTS <= GROUP_THREADS: thread x holds expert x
    const int c = tid < n_exp ? s_cnt[tid] : 0, nt = (c + tile_m - 1) / tile_m;
    int rows_total, tiles_total;
    const int first = group_scan(c, s_wave, rows_total);
    const int tile0 = group_scan(nt, s_wave, tiles_total);
    if (tid < n_exp) {
        for (int j = 0; j < nt; j++) {
            tiles[1 + 3 * (tile0 + j)] = tid;
            tiles[2 + 3 * (tile0 + j)] = first + j * tile_m;
            tiles[3 + 3 * (tile0 + j)] = c - j * tile_m < tile_m ? c - j * tile_m : tile_m;
        }
        s_cnt[tid] = first;
    }
    if (tid == 0) tiles[0] = tiles_total;
    __syncthreads();
    for (int i = tid; i < m * top_k; i += GROUP_THREADS) {
        const int t = i / top_k, k = i % top_k, n = C[t];
        if (k >= n) continue;
        const int *pick = E + (size_t)t * top_k;
        const int x = pick[k];
        const int row = atomicAdd(&s_cnt[x], 1);
        const float w = weights[i];
        row_token[row] = t;
        row_weight[row] = w;
        int o = 0;  // the pick's place in expert order (ties: pick order)
        for (int j = 0; j < n; j++) o += pick[j] < x || (pick[j] == x && j < k);
        pos[(size_t)t * top_k + o] = row;
        wpos[(size_t)t * top_k + o] = w;
    }
}

// out[t] = base[t] (or 0), then + w * y[row] over token t's picks in expert
// order (the mix order, ffn.rs:775-805): pick k's row is pos[t * top_k + k]
// (in expert order, as group_kernel writes it) or, `pos` null, t * top_k + k
// (the picks already in expert order); weights in the same order.  Grid:
// (hidden / 256, tokens).  Every slot's row and weight are loaded together
// with the pick count, not after it (a slot past the count holds a stale
// row, clamped into the `rows` rows of y, whose product is left out of the
// sum), so the value loads wait on one round trip, not two.
__global__ __launch_bounds__(256) void combine_kernel(const float *base, const float *y, const float *weights,
                                                     const int32_t *count, const int32_t *pos, int top_k, int hidden,
                                                     int rows, float *out) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    int pr[MAX_TOPK];
    float pw[MAX_TOPK];
#pragma unroll
    for (int k = 0; k < MAX_TOPK; k++) {
        const bool ok = k < top_k;
        const int r = ok ? (pos ? pos[(size_t)t * top_k + k] : t * top_k + k) : 0;
        pr[k] = min(max(r, 0), rows - 1);
        pw[k] = ok ? weights[(size_t)t * top_k + k] : 0.0f;
    }
    const int n = count[t];
    if (i >= hidden) return;
    float yv[MAX_TOPK];
#pragma unroll
    for (int k = 0; k < MAX_TOPK; k++) yv[k] = k < top_k ? y[(size_t)pr[k] * hidden + i] : 0.0f;
    float v = base ? base[(size_t)t * hidden + i] : 0.0f;
#pragma unroll
    for (int k = 0; k < MAX_TOPK; k++) {
        if (k < n) {
            const float p = pw[k] * yv[k];
            v = v + p;
        }
    }
    out[(size_t)t * hidden + i] = v;
}

size_t up256(size_t n) { return (n + 255) / 256 * 256; }

// Bump allocator over the context's MoE workspace.
struct Carve {
    char *base;
    size_t used = 0;
    template <typename T>
    T *take(size_t n) {
        T *p = reinterpret_cast<T *>(base + used);
        used += up256(n * sizeof(T));
        return p;
    }
};

QAct take_qact(Carve &c, size_t m, size_t k) {
    QAct q;
    q.qs = c.take<int8_t>(m * k);
    q.scales = c.take<float>(m * k / BLOCK);
    q.sums = c.take<int32_t>(m * k / BLOCK);
    return q;
}

int upload_tables(kh_ctx *ctx, kh_moe *moe) {
    if (!moe->dirty) return KH_OK;
    const size_t n = moe->n_experts;
    std::vector<void *> tab(3 * n);
    std::vector<float *> stab(3 * n);
    for (size_t x = 0; x < n; x++) {
        const kh_weight *w[3] = {moe->gate[x], moe->up[x], moe->down[x]};
        for (int j = 0; j < 3; j++) {
            tab[j * n + x] = w[j]->qs;
            stab[j * n + x] = w[j]->scales;
        }
    }
    KH_HIP(hipMemcpyAsync(moe->tab, tab.data(), sizeof(void *) * 3 * n, hipMemcpyHostToDevice, ctx->stream));
    KH_HIP(hipMemcpyAsync(moe->stab, stab.data(), sizeof(float *) * 3 * n, hipMemcpyHostToDevice, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    moe->dirty = false;
    return KH_OK;
}

RouteArgs route_args(const kh_moe *moe, const float *logits, int32_t *experts, float *weights, int32_t *count) {
    RouteArgs r{};
    r.logits = logits;
    r.bias = moe->bias;
    r.n = (int)moe->n_experts;
    r.top_k = (int)moe->top_k;
    r.scoring = moe->scoring;
    r.select = moe->select;
    r.n_group = (int)moe->n_group;
    r.topk_group = (int)moe->topk_group;
    r.norm_topk = moe->norm_topk;
    r.always_scale = moe->select == 2;  // noaux_tc scales always (ffn.rs:251)
    r.scale = moe->scale;
    r.experts = experts;
    r.weights = weights;
    r.count = count;
    return r;
}

GemvJob expert_job(const kh_moe *moe, int which, const int32_t *sel, const float *xf, const float *xf2, float *y) {
    const size_t n = moe->n_experts;
    const kh_weight *w0 = which == 0 ? moe->gate[0] : which == 1 ? moe->up[0] : moe->down[0];
    GemvJob j{};
    j.wtab = const_cast<const void *const *>(moe->tab + which * n);
    j.wstab = const_cast<const float *const *>(moe->stab + which * n);
    j.sel = sel;
    j.xf = xf;
    j.xf2 = xf2;
    j.y = y;
    j.rows = (int)w0->rows;
    j.cols = (int)w0->cols;
    return j;
}

GemvJob plain_job(const kh_weight *w, const float *xf, const float *xf2, float *y) {
    GemvJob j{};
    j.w = w->qs;
    j.ws = w->scales;
    j.xf = xf;
    j.xf2 = xf2;
    j.y = y;
    j.rows = (int)w->rows;
    j.cols = (int)w->cols;
    return j;
}

// One token: decode_together (ffn.rs:820-842) after early() (ffn.rs:556-612).
// One token's buffers in the MoE workspace.
struct DecodeBufs {
    float *logits, *sg, *su;
    int32_t *pe, *cnt, *se;  // picks by rank, their count, picks in expert order
    float *pw, *sw;
    float *g, *u, *y, *ys;   // per pick in expert order; the shared expert's output
};

DecodeBufs decode_bufs(kh_ctx *ctx, const kh_moe *moe) {
    const size_t n = moe->n_experts, k = moe->top_k, hid = moe->hidden, inter = moe->inter;
    const size_t sh = moe->sgate ? moe->sgate->rows : 0;
    Carve c{static_cast<char *>(ctx->moe.ptr)};
    DecodeBufs b;
    b.logits = c.take<float>(n);
    b.sg = c.take<float>(sh ? sh : 1), b.su = c.take<float>(sh ? sh : 1);
    b.pe = c.take<int32_t>(k), b.cnt = c.take<int32_t>(1), b.se = c.take<int32_t>(k);
    b.pw = c.take<float>(k), b.sw = c.take<float>(k);
    b.g = c.take<float>(k * inter), b.u = c.take<float>(k * inter);
    b.y = c.take<float>(k * hid), b.ys = c.take<float>(hid);
    return b;
}

int moe_decode(kh_ctx *ctx, kh_moe *moe, const float *x, float *out) {
    const size_t k = moe->top_k, hid = moe->hidden, inter = moe->inter;
    const size_t sh = moe->sgate ? moe->sgate->rows : 0;
    const DecodeBufs b = decode_bufs(ctx, moe);
    float *logits = b.logits, *sg = b.sg, *su = b.su, *pw = b.pw, *sw = b.sw, *g = b.g, *u = b.u, *y = b.y,
          *ys = b.ys;
    int32_t *pe = b.pe, *cnt = b.cnt, *se = b.se;

    // (1) the router and the shared expert's gate and up read x together
    std::vector<const kh_weight *> w{moe->router};
    std::vector<const float *> xs{x};
    std::vector<float *> ys1{logits};
    if (sh) {
        w.push_back(moe->sgate), xs.push_back(x), ys1.push_back(sg);
        w.push_back(moe->sup), xs.push_back(x), ys1.push_back(su);
    }
    int rc;
    RouteArgs r = route_args(moe, logits, pe, pw, cnt);
    r.sorted_experts = se;
    r.sorted_weights = sw;
    r.arrivals = moe->arrivals;
    // (1) + (2) in one launch where the GEMV has a routing build for it: the
    // router's one workgroup routes its own logits while the shared expert's
    // rows stream (q8, inputs the kernel stages itself)
    bool routed = false;
    if (moe->router->precision == KH_Q8 && !dequant_selected()) {
        bool plain = true;
        for (const kh_weight *v : w) plain = plain && v->precision == KH_Q8 && v->cols <= fuse_max_cols(KH_Q8);
        if (plain) {
            std::vector<GemvJob> j1;
            for (size_t i = 0; i < w.size(); i++) j1.push_back(plain_job(w[i], xs[i], nullptr, ys1[i]));
            rc = launch_gemv_route(ctx, KH_Q8, j1.data(), (int)j1.size(), 0, r);
            if (rc != KH_OK && rc != KH_DECLINED) return rc;
            routed = rc == KH_OK;
        }
    }
    if (!routed) {
        if (moe->router->precision == KH_F32) {  // matvec_many declines f32: run the router alone
            if ((rc = matvec_device(ctx, moe->router, x, nullptr, logits, nullptr))) return rc;
            if (sh && (rc = matvec_many_device(ctx, w.size() - 1, w.data() + 1, xs.data() + 1, ys1.data() + 1)))
                return rc;
        } else if ((rc = matvec_many_device(ctx, w.size(), w.data(), xs.data(), ys1.data()))) {
            return rc;
        }
        // (2) the router
        if ((rc = launch_route(ctx, r, 1))) return rc;
    }
    // (3) every chosen expert's gate and up, through the device tables
    std::vector<GemvJob> jobs;
    for (size_t i = 0; i < k; i++) {
        jobs.push_back(expert_job(moe, 0, se + i, x, nullptr, g + i * inter));
        jobs.push_back(expert_job(moe, 1, se + i, x, nullptr, u + i * inter));
    }
    if ((rc = launch_gemv(ctx, moe->precision, jobs.data(), (int)jobs.size()))) return rc;
    // (4) every down projection, input swiglu(gate, up) staged by the kernel
    jobs.clear();
    for (size_t i = 0; i < k; i++) jobs.push_back(expert_job(moe, 2, se + i, g + i * inter, u + i * inter, y + i * hid));
    if (sh && moe->sdown->precision == moe->precision) jobs.push_back(plain_job(moe->sdown, sg, su, ys));
    if ((rc = launch_gemv(ctx, moe->precision, jobs.data(), (int)jobs.size()))) return rc;
    if (sh && moe->sdown->precision != moe->precision) {
        GemvJob j = plain_job(moe->sdown, sg, su, ys);
        if ((rc = launch_gemv(ctx, moe->sdown->precision, &j, 1))) return rc;
    }
    // (5) out = shared, then + w * y in expert order
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((hid + 255) / 256), 1), dim3(256), 0, ctx->stream,
                       sh ? ys : nullptr, y, sw, cnt, nullptr, (int)k, (int)hid, (int)k, out);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

// Ffn::run over pre-quantised rows with a plain (ungrouped) weight set.
int ffn_rows(kh_ctx *ctx, const kh_weight *gate, const kh_weight *up, const kh_weight *down, const QAct &xq,
             size_t m, float *g, float *u, const QAct &hq, float *y) {
    GemmArgs a{};
    a.xq = xq.qs, a.xs = xq.scales, a.xsum = xq.sums;
    a.M = (int)m, a.K = (int)gate->cols;
    int tn;
    const int tm = gemm_tiles(ctx, (int)m, (int)gate->rows, &tn);
    int rc;
    a.w = gate->qs, a.ws = gate->scales, a.N = (int)gate->rows, a.y = g;
    if (gate->precision == up->precision && gate->rows == up->rows && gate->cols == up->cols) {
        // gate and up in one launch over the same activation tiles
        a.w2 = up->qs, a.ws2 = up->scales, a.y2 = u;
        if ((rc = plan_split(ctx, a, tm, tn)) || (rc = launch_gemm_q(ctx, gate->precision, a, 0, tm, tn))) return rc;
    } else {
        if ((rc = plan_split(ctx, a, tm, tn)) || (rc = launch_gemm_q(ctx, gate->precision, a, 0, tm, tn))) return rc;
        a.w = up->qs, a.ws = up->scales, a.N = (int)up->rows, a.y = u;
        if ((rc = plan_split(ctx, a, tm, tn)) || (rc = launch_gemm_q(ctx, up->precision, a, 0, tm, tn))) return rc;
    }
    if ((rc = launch_swiglu_qact(ctx, g, u, m, gate->rows, hq))) return rc;
    GemmArgs d{};
    d.xq = hq.qs, d.xs = hq.scales, d.xsum = hq.sums;
    d.M = (int)m, d.K = (int)down->cols, d.N = (int)down->rows;
    d.w = down->qs, d.ws = down->scales, d.y = y;
    int tdn;
    const int td = gemm_tiles(ctx, (int)m, (int)down->rows, &tdn);
    if ((rc = plan_split(ctx, d, td, tdn))) return rc;
    return launch_gemm_q(ctx, down->precision, d, 0, td, tdn);
}

// A batch: Moe::run for m > 1 (ffn.rs:615-708, mix ffn.rs:788-805).
// A batch's buffers in the MoE workspace.  Rows are the picks grouped by
// expert; pos / wpos give each token's rows and weights in expert order.
struct PrefillBufs {
    float *logits;
    int32_t *pe, *cnt, *pos;
    float *pw, *wpos;
    int32_t *row_token, *tiles;
    float *row_weight;
    QAct hq;
    float *g, *u;
    QAct rq;                     // swiglu(g, u) per row, quantised
    float *y;
    float *base, *sg, *su;       // the shared expert (null without one)
    QAct sq;
};

size_t prefill_max_tiles(size_t total, size_t n, int tile_m) { return (total + tile_m - 1) / tile_m + n; }

PrefillBufs prefill_bufs(kh_ctx *ctx, const kh_moe *moe, size_t m) {
    const size_t n = moe->n_experts, k = moe->top_k, hid = moe->hidden, inter = moe->inter;
    const size_t sh = moe->sgate ? moe->sgate->rows : 0;
    const size_t total = m * k, max_tiles = prefill_max_tiles(total, n, 32);
    Carve c{static_cast<char *>(ctx->moe.ptr)};
    PrefillBufs b{};
    b.logits = c.take<float>(m * n);
    b.pe = c.take<int32_t>(total), b.cnt = c.take<int32_t>(m), b.pos = c.take<int32_t>(total);
    b.pw = c.take<float>(total), b.wpos = c.take<float>(total);
    b.row_token = c.take<int32_t>(total), b.tiles = c.take<int32_t>(1 + 3 * max_tiles);
    b.row_weight = c.take<float>(total);
    b.hq = take_qact(c, m, hid);
    b.g = c.take<float>(total * inter), b.u = c.take<float>(total * inter);
    b.rq = take_qact(c, total, inter);
    b.y = c.take<float>(total * hid);
    if (sh) {
        b.base = c.take<float>(m * hid);
        b.sg = c.take<float>(m * sh);
        b.su = c.take<float>(m * sh);
        b.sq = take_qact(c, m, sh);
    }
    return b;
}

// route_rows_kernel for m tokens quantised in q against a q8 router; KH_DECLINED
// where it is not built for the router (other precisions, rows past 256
// blocks, limits route_one does not take, KVAD_DEQUANT).
int launch_route_rows(kh_ctx *ctx, const RouteArgs &r, float *logits, const QAct &q, const kh_weight *router, size_t m) {
    const size_t cols = router->cols, nb = cols / BLOCK;
    if (router->precision != KH_Q8 || cols % BLOCK || nb > 256 || router->rows != (size_t)r.n ||
        dequant_selected() || r.n > MAX_EXPERTS ||
        r.top_k > MAX_TOPK || r.n_group > MAX_GROUPS || m > 0x7fffffff)
        return KH_DECLINED;
    const dim3 grid((unsigned)m);
    const int8_t *wq = static_cast<const int8_t *>(router->qs);
    if (nb <= 64)
        hipLaunchKernelGGL(route_rows_kernel<1>, grid, dim3(256), 0, ctx->stream, r, logits, q.qs, q.scales, wq,
                           router->scales, (int)cols);
    else if (nb <= 128)
        hipLaunchKernelGGL(route_rows_kernel<2>, grid, dim3(256), 0, ctx->stream, r, logits, q.qs, q.scales, wq,
                           router->scales, (int)cols);
    else
        hipLaunchKernelGGL(route_rows_kernel<4>, grid, dim3(256), 0, ctx->stream, r, logits, q.qs, q.scales, wq,
                           router->scales, (int)cols);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int moe_prefill(kh_ctx *ctx, kh_moe *moe, const float *hs, size_t m, float *out) {
    const size_t n = moe->n_experts, k = moe->top_k, hid = moe->hidden, inter = moe->inter;
    const size_t sh = moe->sgate ? moe->sgate->rows : 0;
    const size_t total = m * k;
    const int forced = env_int("KVAD_MOE_TILE_M", 0);  // tuning knob: rows per expert tile (32 / 64)
    // 64-row tiles once experts average 32 rows: an expert's weights are
    // then read by fewer tiles (measured at DeepSeek-V2-Lite's 48 rows a
    // expert: 477 against 501 us a layer)
    const int tile_m = forced == 32 || forced == 64 ? forced : total / n >= 32 ? 64 : 32;
    const size_t max_tiles = prefill_max_tiles(total, n, tile_m);
    const PrefillBufs b = prefill_bufs(ctx, moe, m);
    float *logits = b.logits, *pw = b.pw, *wpos = b.wpos, *row_weight = b.row_weight, *g = b.g, *u = b.u,
          *y = b.y, *base = b.base, *sg = b.sg, *su = b.su;
    int32_t *pe = b.pe, *cnt = b.cnt, *pos = b.pos, *row_token = b.row_token, *tiles = b.tiles;
    const QAct hq = b.hq, rq = b.rq, sq = b.sq;
    int rc;
    // the activations, quantised once for the router, every expert and the
    // shared one (QActBatch::new, quant.rs:693-714)
    if ((rc = launch_qact(ctx, hs, m, hid, hq))) return rc;
    // router logits (any precision; quantised weights read the codes above,
    // the ones matmul_bt would make), then the routes: for q8 routers one
    // launch, a workgroup per token
    const RouteArgs ra = route_args(moe, logits, pe, pw, cnt);
    rc = launch_route_rows(ctx, ra, logits, hq, moe->router, m);
    if (rc == KH_DECLINED) {
        if (moe->router->precision != KH_F32 && moe->router->cols == hid)
            rc = launch_matmul_q(ctx, moe->router, hq, m, nullptr, logits, 0);
        else
            rc = matmul_device(ctx, moe->router, hs, m, nullptr, logits);
        if (!rc) rc = launch_route(ctx, ra, (int)m);
    }
    if (rc) return rc;
    // by_expert, and the tiles of the grouped GEMMs
    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(GROUP_THREADS), 0, ctx->stream, pe, pw, cnt, (int)m, (int)k,
                       (int)n, tile_m, row_token, row_weight, pos, wpos, tiles);
    KH_HIP(hipGetLastError());
    // the shared expert on every token (SharedExpert::run, ffn.rs:437-451)
    if (sh && (rc = ffn_rows(ctx, moe->sgate, moe->sup, moe->sdown, hq, m, sg, su, sq, base))) return rc;
    // each expert's gate and up over its own rows
    GemmArgs a{};
    a.xq = hq.qs, a.xs = hq.scales, a.xsum = hq.sums;
    a.M = (int)m, a.K = (int)hid, a.N = (int)inter;
    a.tiles = tiles, a.gather = row_token;
    a.wtab = const_cast<const void *const *>(moe->tab);
    a.wstab = const_cast<const float *const *>(moe->stab);
    a.y = g;
    // and up in the same launch (the second weight table)
    a.wtab2 = const_cast<const void *const *>(moe->tab + n);
    a.wstab2 = const_cast<const float *const *>(moe->stab + n);
    a.y2 = u;
    if ((rc = launch_gemm_q(ctx, moe->precision, a, (int)max_tiles, tile_m))) return rc;
    if ((rc = launch_swiglu_qact(ctx, g, u, total, inter, rq))) return rc;
    // each expert's down over its rows of swiglu(gate, up)
    GemmArgs d{};
    d.xq = rq.qs, d.xs = rq.scales, d.xsum = rq.sums;
    d.M = (int)total, d.K = (int)inter, d.N = (int)hid;
    d.tiles = tiles;
    d.wtab = const_cast<const void *const *>(moe->tab + 2 * n);
    d.wstab = const_cast<const float *const *>(moe->stab + 2 * n);
    d.y = y;
    if ((rc = launch_gemm_q(ctx, moe->precision, d, (int)max_tiles, tile_m))) return rc;
    // out = shared, then + w * y per token in expert order
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((hid + 255) / 256), (unsigned)m), dim3(256), 0, ctx->stream,
                       base, y, wpos, cnt, pos, (int)k, (int)hid, (int)total, out);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

size_t workspace_bytes(const kh_moe *moe, size_t m) {
    const size_t n = moe->n_experts, k = moe->top_k, hid = moe->hidden, inter = moe->inter;
    const size_t sh = moe->sgate ? moe->sgate->rows : 0;
    const size_t total = m * k, max_tiles = prefill_max_tiles(total, n, 32);
    auto q = [](size_t a, size_t b) { return up256(a * b) + 2 * up256(4 * a * b / BLOCK); };
    size_t b = up256(4 * m * n) + 6 * up256(4 * total) + up256(4 * m) + up256(4 * (1 + 3 * max_tiles));
    b += q(m, hid) + 2 * up256(4 * total * inter) + q(total, inter) + up256(4 * total * hid);
    b += sh ? up256(4 * m * hid) + 2 * up256(4 * m * sh) + q(m, sh) : 0;
    b += up256(4 * hid) + 2 * up256(4 * (sh ? sh : 1)) + 4 * up256(4 * k) + up256(4 * k * hid);  // decode extras
    return b + 4096;
}

}  // namespace

int launch_route(kh_ctx *ctx, const RouteArgs &r, int m) {
    if (r.n > MAX_EXPERTS || r.top_k > MAX_TOPK || r.n_group > MAX_GROUPS)
        return fail(KH_DECLINED, "route: more experts, picks or groups than the device router takes");
    if (m == 0) return KH_OK;
    hipLaunchKernelGGL(route_kernel, dim3((unsigned)m), dim3(64), 0, ctx->stream, r);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int moe_run_device(kh_ctx *ctx, kh_moe *moe, const float *hs, size_t m, float *out) {
    if (!moe->router) return fail(KH_EINVAL, "moe: no router set");
    for (size_t x = 0; x < moe->n_experts; x++)
        if (!moe->gate[x] || !moe->up[x] || !moe->down[x]) return fail(KH_EINVAL, "moe: an expert is not set");
    if (m == 0) return KH_OK;
    int rc = upload_tables(ctx, moe);
    if (rc) return rc;
    if ((rc = ensure(ctx, ctx->moe, workspace_bytes(moe, m)))) return rc;
    return m == 1 ? moe_decode(ctx, moe, hs, out) : moe_prefill(ctx, moe, hs, m, out);
}

int route_device(kh_ctx *ctx, const kh_moe *moe, const float *logits, size_t m, int32_t *experts, float *weights,
                 int32_t *count) {
    return launch_route(ctx, route_args(moe, logits, experts, weights, count), (int)m);
}

int moe_picks(kh_ctx *ctx, const kh_moe *moe, size_t m, const MoePicks &o) {
    const size_t n = moe->n_experts, k = moe->top_k, hid = moe->hidden, inter = moe->inter;
    const size_t sh = moe->sgate ? moe->sgate->rows : 0, total = m * k;
    if (m == 0) return KH_OK;
    if (!ctx->moe.ptr || ctx->moe.bytes < workspace_bytes(moe, m))
        return fail(KH_EINVAL, "moe picks: no run of this many tokens to read");
    KH_HIP(hipStreamSynchronize(ctx->stream));
    auto get = [&](const void *src, size_t bytes) {
        std::vector<char> h(bytes);
        if (bytes && hipMemcpy(h.data(), src, bytes, hipMemcpyDeviceToHost) != hipSuccess) h.clear();
        return h;
    };
    auto f32 = [](const std::vector<char> &h) { return reinterpret_cast<const float *>(h.data()); };
    auto i32 = [](const std::vector<char> &h) { return reinterpret_cast<const int32_t *>(h.data()); };
    // per token: its count, then for pick j (expert order) the expert, the
    // weight and the row holding its gate / up / hidden / output
    std::vector<int32_t> cnt(m), expert(total, 0), row(total, -1);
    std::vector<float> weight(total, 0.0f);
    const float *g_d, *u_d, *y_d, *logits_d, *sg_d = nullptr, *su_d = nullptr, *ys_d = nullptr;
    QAct rq{};
    if (m == 1) {
        const DecodeBufs b = decode_bufs(ctx, moe);
        auto c = get(b.cnt, 4), e = get(b.se, 4 * k), w = get(b.sw, 4 * k);
        if (c.empty() || e.empty() || w.empty()) return fail(KH_EINVAL, "moe picks: copy failed");
        cnt[0] = i32(c)[0];
        for (size_t j = 0; j < k; j++)
            if ((int)j < cnt[0]) expert[j] = i32(e)[j], weight[j] = f32(w)[j], row[j] = (int)j;
        g_d = b.g, u_d = b.u, y_d = b.y, logits_d = b.logits;
        if (sh) sg_d = b.sg, su_d = b.su, ys_d = b.ys;
    } else {
        const PrefillBufs b = prefill_bufs(ctx, moe, m);
        auto c = get(b.cnt, 4 * m), e = get(b.pe, 4 * total), p = get(b.pos, 4 * total), w = get(b.wpos, 4 * total);
        if (c.empty() || e.empty() || p.empty() || w.empty()) return fail(KH_EINVAL, "moe picks: copy failed");
        for (size_t t = 0; t < m; t++) {
            cnt[t] = i32(c)[t];
            std::vector<int32_t> xs(i32(e) + t * k, i32(e) + t * k + cnt[t]);
            std::sort(xs.begin(), xs.end());
            for (int j = 0; j < cnt[t]; j++) {
                expert[t * k + j] = xs[j];
                row[t * k + j] = i32(p)[t * k + j];
                weight[t * k + j] = f32(w)[t * k + j];
            }
        }
        g_d = b.g, u_d = b.u, y_d = b.y, logits_d = b.logits, rq = b.rq;
        if (sh) sg_d = b.sg, su_d = b.su, ys_d = b.base;
    }
    if (o.count) std::copy(cnt.begin(), cnt.end(), o.count);
    if (o.experts) std::copy(expert.begin(), expert.end(), o.experts);
    if (o.weights) std::copy(weight.begin(), weight.end(), o.weights);
    if (o.logits) KH_HIP(hipMemcpy(o.logits, logits_d, 4 * m * n, hipMemcpyDeviceToHost));
    // the rows, gathered pick by pick (an unused pick's stay zero)
    auto gather = [&](void *dst, const void *src, size_t row_bytes) -> int {
        if (!dst) return KH_OK;
        memset(dst, 0, total * row_bytes);
        for (size_t i = 0; i < total; i++)
            if (row[i] >= 0)
                KH_HIP(hipMemcpy(static_cast<char *>(dst) + i * row_bytes,
                                 static_cast<const char *>(src) + (size_t)row[i] * row_bytes, row_bytes,
                                 hipMemcpyDeviceToHost));
        return KH_OK;
    };
    int rc;
    if ((rc = gather(o.gate, g_d, 4 * inter)) || (rc = gather(o.up, u_d, 4 * inter)) ||
        (rc = gather(o.out, y_d, 4 * hid)))
        return rc;
    if (o.hidden_qs || o.hidden_scales) {
        if (m == 1) return fail(KH_DECLINED, "moe picks: one token's hidden codes stay inside the down GEMV");
        if ((rc = gather(o.hidden_qs, rq.qs, inter)) || (rc = gather(o.hidden_scales, rq.scales, 4 * inter / BLOCK)))
            return rc;
    }
    if (sh) {
        if (o.shared_gate) KH_HIP(hipMemcpy(o.shared_gate, sg_d, 4 * m * sh, hipMemcpyDeviceToHost));
        if (o.shared_up) KH_HIP(hipMemcpy(o.shared_up, su_d, 4 * m * sh, hipMemcpyDeviceToHost));
        if (o.shared_out) KH_HIP(hipMemcpy(o.shared_out, ys_d, 4 * m * hid, hipMemcpyDeviceToHost));
    }
    return KH_OK;
}

}  // namespace kh
