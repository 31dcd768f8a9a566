// A device-resident decoder session for the Llama family (Qwen2/2.5/3 dense,
// Llama): the forward of one token (crates/llm/src/model/llama.rs:224-289
// run_rows with m = 1, embed and head at :384-415) with every operator on
// the device, the KV cache in HBM, and the greedy next token chosen on the
// device (sampler::argmax, crates/llm/src/sampler.rs:217-226).
//
// The position and the token live in device memory, so one token's launches
// are the same every step: `kh_llm_generate` captures them once as a HIP
// graph and replays it per token.  Per layer: q/k/v (+bias) as one GEMV
// launch with the RMSNorm staged by the GEMV; attention over the cache, its
// length read from the device, with RoPE of q and k (per-head RMSNorm first
// where the model has q/k norms) and the push of k and v into the cache row
// done by the attention's own split kernel; o as a GEMV that adds into the
// residual; gate and up as one launch, RMSNorm staged; down with
// swiglu(gate, up) staged by the GEMV and added into the residual.
#include <algorithm>
#include <initializer_list>
#include <memory>

#include "common.hpp"
#include "device.hpp"

namespace kh {
namespace {

// sampler::argmax (sampler.rs:217-226): the first of equal maxima; a NaN
// never wins, and a NaN first entry keeps index 0.  Two launches: each
// workgroup reduces a run of entries 1.. (largest, then lowest index), then
// one workgroup reduces the runs, compares with entry 0, and makes the next
// token the input, advances the position and records the step's token.
constexpr int ARGMAX_BLOCKS = 256;
constexpr int ARGMAX_CAP = 16384;  // greedy partials the head GEMV's workgroups may write

__device__ __forceinline__ void better(float &bv, int &bi, float ov, int oi) {
    if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) bv = ov, bi = oi;
}

__device__ void block_best(float &bv, int &bi, float *s_v, int *s_i) {
    const int t = threadIdx.x;
    s_v[t] = bv;
    s_i[t] = bi;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w) {
            float v = s_v[t];
            int i = s_i[t];
            better(v, i, s_v[t + w], s_i[t + w]);
            s_v[t] = v, s_i[t] = i;
        }
        __syncthreads();
    }
    bv = s_v[0], bi = s_i[0];
}

// Row blockIdx.y of v [rows][n]: partials [rows][ARGMAX_BLOCKS].
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *v, int n, float *pv, int *pi) {
    __shared__ float s_v[256];
    __shared__ int s_i[256];
    v += (size_t)blockIdx.y * n;
    pv += (size_t)blockIdx.y * ARGMAX_BLOCKS;
    pi += (size_t)blockIdx.y * ARGMAX_BLOCKS;
    const int per = (n - 1 + ARGMAX_BLOCKS - 1) / ARGMAX_BLOCKS;
    const int lo = 1 + blockIdx.x * per, hi = min(n, lo + per);
    float bv = -INFINITY;
    int bi = -1;
    for (int i = lo + threadIdx.x; i < hi; i += 256) {
        const float x = v[i];
        if (x == x) better(bv, bi, x, i);
    }
    block_best(bv, bi, s_v, s_i);
    if (threadIdx.x == 0) pv[blockIdx.x] = bv, pi[blockIdx.x] = bi;
}

// Entry 0 against the best of entries 1..: the first of equal maxima wins.
__device__ __forceinline__ int pick(const float *v, int n, float bv, int bi) {
    const float first = n > 0 ? v[0] : 0.0f;
    return n > 1 && first == first && bi >= 0 && bv > first ? bi : 0;
}

// One workgroup per row of v [rows][n]: next[row].
__global__ __launch_bounds__(256) void argmax_rows_kernel(const float *v, int n, const float *pv, const int *pi,
                                                         int32_t *next) {
    __shared__ float s_v[256];
    __shared__ int s_i[256];
    const int row = blockIdx.x;
    float bv = pv[(size_t)row * ARGMAX_BLOCKS + threadIdx.x];
    int bi = pi[(size_t)row * ARGMAX_BLOCKS + threadIdx.x];
    block_best(bv, bi, s_v, s_i);
    if (threadIdx.x == 0) next[row] = pick(v + (size_t)row * n, n, bv, bi);
}

// The embedding the next step starts from: the chosen token's row of the
// embedding weight (Weight::row, llama.rs:384-391).
struct NextEmbed {
    int prec;
    const void *qs;
    const float *scales;
    size_t cols;
    float *x;
};

// The step's end as a launch of its own (f32 heads, KVAD_HEAD_TAIL=0; the
// head GEMV's greedy_tail otherwise).  The partials' count is *pn (the head
// GEMV's workgroups) or, without pn, ARGMAX_BLOCKS (argmax_partial_kernel).  The chosen token becomes the next
// input, the position advances, the step is recorded, and the token's
// embedding row is written to e.x, so a captured step needs no launch of its
// own for it.
__global__ __launch_bounds__(256) void argmax_final_kernel(const float *v, int n, const float *pv, const int *pi,
                                                          const int *pn, int32_t *token, int32_t *pos, int32_t *step,
                                                          int32_t *out, int out_cap, NextEmbed e) {
    __shared__ float s_v[256];
    __shared__ int s_i[256];
    __shared__ int s_best;
    const int np = pn ? min(*pn, ARGMAX_CAP) : ARGMAX_BLOCKS;
    float bv = -INFINITY;
    int bi = -1;
    for (int t0 = 0; t0 < np; t0 += 8 * 256) {  // eight loads in flight per thread
        float v8[8];
        int i8[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int t = t0 + u * 256 + (int)threadIdx.x;
            v8[u] = t < np ? pv[t] : -INFINITY;
            i8[u] = t < np ? pi[t] : -1;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) better(bv, bi, v8[u], i8[u]);
    }
    block_best(bv, bi, s_v, s_i);
    if (threadIdx.x == 0) {
        const int best = pick(v, n, bv, bi);
        s_best = best;
        *token = best;
        *pos = *pos + 1;
        const int k = *step;
        if (out && k < out_cap) out[k] = best;
        *step = k + 1;
    }
    __syncthreads();
    const size_t r = (size_t)s_best;
    for (size_t k = threadIdx.x; k < e.cols; k += 256) e.x[k] = dev::dequant_elem(e.prec, e.qs, e.scales, e.cols, r, k);
}

template <typename T>
int dev_alloc(T **p, size_t n) {
    KH_HIP(hipMalloc(reinterpret_cast<void **>(p), sizeof(T) * (n ? n : 1)));
    return KH_OK;
}

int dev_vector(float **p, const float *host, size_t n) {
    if (!host) {
        *p = nullptr;
        return KH_OK;
    }
    int rc = dev_alloc(p, n);
    if (rc) return rc;
    KH_HIP(hipMemcpy(*p, host, 4 * n, hipMemcpyHostToDevice));
    return KH_OK;
}

GemvJob gemv_job(const kh_weight *w, const float *x, const float *x2, const float *bias, float *y, int acc) {
    GemvJob j{};
    j.w = w->qs;
    j.ws = w->scales;
    j.xf = x;
    j.xf2 = x2;
    j.bias = bias;
    j.y = y;
    j.rows = (int)w->rows;
    j.cols = (int)w->cols;
    j.accumulate = acc;
    return j;
}

// Jobs of one precision in one launch; mixed precisions in as many.
int run_jobs(kh_ctx *ctx, const std::vector<std::pair<const kh_weight *, GemvJob>> &jobs) {
    for (int prec : {KH_Q8, KH_Q4, KH_Q4K, KH_F32}) {
        std::vector<GemvJob> js;
        for (auto &j : jobs)
            if (j.first->precision == prec) js.push_back(j.second);
        if (!js.empty()) {
            int rc = launch_gemv(ctx, prec, js.data(), (int)js.size());
            if (rc) return rc;
        }
    }
    return KH_OK;
}

// The quantised GEMV can take swiglu(gate, up) as its input when it stages
// the activation itself; the f32 GEMV reads its input as it is.
bool fusable(const kh_weight *w) { return w->precision != KH_F32 && w->cols <= fuse_max_cols(w->precision); }

// The GEMV can take rms_norm(x) as its input when it stages x itself.
bool norm_fusable(const kh_weight *w) { return w->precision != KH_F32 && w->cols <= fuse_max_cols(w->precision); }

GemvJob normed(GemvJob j, bool fuse, const float *w, float eps) {
    if (fuse) j.norm_w = w, j.norm_eps = eps;
    return j;
}

// Jobs whose shared f32 input x (n wide) is too wide for the quantised
// GEMV to stage itself: x is quantised first into m->hq
// (QActivation::new, quant.rs:1037-1067) and those jobs read the codes.
int wide_input(kh_ctx *ctx, kh_llm *m, std::vector<std::pair<const kh_weight *, GemvJob>> &jobs, const float *x,
               size_t n) {
    bool wide = false;
    for (auto &j : jobs) wide |= j.first->precision != KH_F32 && n > fuse_max_cols(j.first->precision);
    if (!wide) return KH_OK;
    const int rc = launch_qact(ctx, x, 1, n, m->hq);
    if (rc) return rc;
    for (auto &j : jobs) {
        if (j.first->precision == KH_F32) continue;
        j.second.xf = nullptr;
        j.second.xq = m->hq.qs, j.second.xs = m->hq.scales, j.second.xsum = m->hq.sums;
    }
    return KH_OK;
}

// A copy of n floats of device memory to the trace's host buffer (null: none).
int trace_copy(kh_ctx *ctx, float *dst, const float *src, size_t n) {
    if (dst) KH_HIP(hipMemcpyAsync(dst, src, 4 * n, hipMemcpyDeviceToHost, ctx->stream));
    return KH_OK;
}

// n rows of `width` floats (src rows packed) to host rows `pitch` floats apart.
int trace_rows(kh_ctx *ctx, float *dst, size_t pitch, const float *src, size_t width, size_t n) {
    KH_HIP(hipMemcpy2DAsync(dst, 4 * pitch, src, 4 * width, 4 * width, n, hipMemcpyDeviceToHost, ctx->stream));
    return KH_OK;
}

int head_step(kh_ctx *ctx, kh_llm *m, const float *x, bool record = true);

// One token's launches, all on the context's stream.  With `embed` the
// step starts from the token's embedding row (llama.rs:384-391); without,
// from the row the previous step's argmax wrote into x (captured steps).
// With a trace (the parity hook kh_debug_llm_trace; never under capture)
// each sub-block's results are copied out as it ends.
int step(kh_ctx *ctx, kh_llm *m, const kh_llm_trace *tr = nullptr, bool embed = true) {
    const kh_llm_spec &s = m->spec;
    const size_t qd = s.n_head * s.head_dim, kvd = s.n_kv_head * s.head_dim;
    int rc;
    if (embed && (rc = launch_dequant_row_dev(ctx, m->embed, m->token, m->x))) return rc;
    if (tr && (rc = trace_copy(ctx, tr->x_embed, m->x, s.n_embd))) return rc;
    for (size_t l = 0; l < s.n_layer; l++) {
        const kh_llm::Layer &L = m->layers[l];
        // ---- attention sub-block (llama.rs:241-276)
        std::vector<std::pair<const kh_weight *, GemvJob>> jobs;
        const bool fq = norm_fusable(L.q) && norm_fusable(L.k) && norm_fusable(L.v);
        const float *qin = fq ? m->x : m->h;
        if (!fq && (rc = launch_rms_norm(ctx, m->x, L.attn_norm, 1, s.n_embd, s.eps, m->h))) return rc;
        jobs.push_back({L.q, normed(gemv_job(L.q, qin, nullptr, L.q_b, m->qkv, 0), fq, L.attn_norm, s.eps)});
        jobs.push_back({L.k, normed(gemv_job(L.k, qin, nullptr, L.k_b, m->qkv + qd, 0), fq, L.attn_norm, s.eps)});
        jobs.push_back(
            {L.v, normed(gemv_job(L.v, qin, nullptr, L.v_b, m->qkv + qd + kvd, 0), fq, L.attn_norm, s.eps)});
        if ((!fq && (rc = wide_input(ctx, m, jobs, m->h, s.n_embd))) || (rc = run_jobs(ctx, jobs))) return rc;
        // attention over the cache, its length read from the device, with the
        // per-head norms, RoPE and the push of k and v fused in
        const AttnRope rp{m->qkv + qd, m->qkv + qd + kvd, m->rope_cos, m->rope_sin, L.q_norm, L.k_norm,
                          s.eps, s.rope_interleaved, 0};
        if ((rc = launch_attend_devlen(ctx, (int)s.n_head, (int)s.n_kv_head, (int)s.head_dim, m->qkv, m->kc[l],
                                       m->vc[l], kvd, kvd, m->pos, 1, m->attn_max, m->att, m->attn_ws, m->attn_ws_bytes, &rp)))
            return rc;
        jobs.clear();
        jobs.push_back({L.o, gemv_job(L.o, m->att, nullptr, nullptr, m->x, 1)});
        if ((rc = wide_input(ctx, m, jobs, m->att, qd)) || (rc = run_jobs(ctx, jobs))) return rc;
        if (tr) {
            const size_t n = m->len + 1;  // positions held after the push
            if ((rc = trace_copy(ctx, tr->qkv ? tr->qkv + l * (qd + 2 * kvd) : nullptr, m->qkv, qd + 2 * kvd)) ||
                (rc = trace_copy(ctx, tr->k_cache ? tr->k_cache + l * n * kvd : nullptr, m->kc[l], n * kvd)) ||
                (rc = trace_copy(ctx, tr->v_cache ? tr->v_cache + l * n * kvd : nullptr, m->vc[l], n * kvd)) ||
                (rc = trace_copy(ctx, tr->att ? tr->att + l * qd : nullptr, m->att, qd)) ||
                (rc = trace_copy(ctx, tr->x_attn ? tr->x_attn + l * s.n_embd : nullptr, m->x, s.n_embd)))
                return rc;
        }
        // ---- MLP sub-block (llama.rs:278-285, Ffn::run ffn.rs:370-375)
        const bool fm = norm_fusable(L.gate) && norm_fusable(L.up);
        const float *min_ = fm ? m->x : m->h;
        if (!fm && (rc = launch_rms_norm(ctx, m->x, L.mlp_norm, 1, s.n_embd, s.eps, m->h))) return rc;
        // gate and up as one SwiGLU-pair job where the rows fit: each pair's
        // swiglu is written once (hsw) and down stages it as it is, in place
        // of every down workgroup recomputing swiglu(gate, up); the same
        // values, so the same codes
        bool paired = false;
        if (fm && L.gate->precision == L.up->precision && L.gate->rows == L.up->rows && L.gate->cols == L.up->cols &&
            gemv_pairs_fit(L.gate->precision, L.gate->cols) && L.down->precision != KH_F32 && fusable(L.down)) {
            GemvJob j = normed(gemv_job(L.gate, min_, nullptr, nullptr, m->g, 0), true, L.mlp_norm, s.eps);
            j.w2 = L.up->qs, j.ws2 = L.up->scales, j.y2 = m->u, j.h = m->hsw;
            j.rows = 2 * (int)L.gate->rows;
            rc = launch_gemv(ctx, L.gate->precision, &j, 1);
            if (rc && rc != KH_DECLINED) return rc;
            paired = rc == KH_OK;
        }
        jobs.clear();
        if (!paired) {
            jobs.push_back({L.gate, normed(gemv_job(L.gate, min_, nullptr, nullptr, m->g, 0), fm, L.mlp_norm, s.eps)});
            jobs.push_back({L.up, normed(gemv_job(L.up, min_, nullptr, nullptr, m->u, 0), fm, L.mlp_norm, s.eps)});
            if ((!fm && (rc = wide_input(ctx, m, jobs, m->h, s.n_embd))) || (rc = run_jobs(ctx, jobs))) return rc;
            jobs.clear();
        }
        if (paired) {  // down over swiglu(gate, up) as staged f32
            jobs.push_back({L.down, gemv_job(L.down, m->hsw, nullptr, nullptr, m->x, 1)});
        } else if (L.down->precision == KH_F32) {  // swiglu_inplace (ffn.rs:386), then the f32 GEMV
            if ((rc = launch_swiglu(ctx, m->g, m->u, s.n_ff))) return rc;
            jobs.push_back({L.down, gemv_job(L.down, m->g, nullptr, nullptr, m->x, 1)});
        } else if (fusable(L.down)) {
            jobs.push_back({L.down, gemv_job(L.down, m->g, m->u, nullptr, m->x, 1)});
        } else {  // too wide to stage in LDS: quantise swiglu(gate, up) first
            if ((rc = launch_swiglu_qact(ctx, m->g, m->u, 1, s.n_ff, m->hq))) return rc;
            GemvJob j = gemv_job(L.down, nullptr, nullptr, nullptr, m->x, 1);
            j.xq = m->hq.qs, j.xs = m->hq.scales, j.xsum = m->hq.sums;
            jobs.push_back({L.down, j});
        }
        if ((rc = run_jobs(ctx, jobs))) return rc;
        if (tr && L.down->precision != KH_F32) {  // (the f32 path leaves swiglu in g)
            if ((rc = trace_copy(ctx, tr->gate ? tr->gate + l * s.n_ff : nullptr, m->g, s.n_ff)) ||
                (rc = trace_copy(ctx, tr->up ? tr->up + l * s.n_ff : nullptr, m->u, s.n_ff)))
                return rc;
        }
        if (tr && (rc = trace_copy(ctx, tr->x_mlp ? tr->x_mlp + l * s.n_embd : nullptr, m->x, s.n_embd))) return rc;
    }
    return head_step(ctx, m, m->x);
}

// The head over the last residual row x (llama.rs:404-411, Transformer::head
// with all = false) into m->logits, then the greedy choice (sampler.rs:217-226):
// the chosen token becomes the next input (its embedding row in m->x), the
// position advances by one and, with `record`, the step's token is written to
// the generated tokens (kh_llm_generate's record; a prompt's pass leaves it).
int head_step(kh_ctx *ctx, kh_llm *m, const float *x, bool record) {
    int32_t *const out = record ? m->out : nullptr;
    const kh_llm_spec &s = m->spec;
    int rc;
    const kh_weight *head = m->head ? m->head : m->embed;
    const bool fh = norm_fusable(head);
    if (!fh && (rc = launch_rms_norm(ctx, x, m->final_norm, 1, s.n_embd, s.eps, m->h))) return rc;
    std::vector<std::pair<const kh_weight *, GemvJob>> jobs{
        {head, normed(gemv_job(head, fh ? x : m->h, nullptr, nullptr, m->logits, 0), fh, m->final_norm, s.eps)}};
    if (!fh && (rc = wide_input(ctx, m, jobs, m->h, s.n_embd))) return rc;
    // the greedy choice (sampler.rs:217-226): each workgroup of the head GEMV
    // keeps its best row, one workgroup then takes the best of them; f32
    // heads, or launches of more workgroups than partials, run a partial pass
    // and a launch of one workgroup
    bool kept = false;
    if (head->precision != KH_F32) {
        // the step ends in the head's last workgroup to finish, with no
        // launch of its own (KVAD_HEAD_TAIL=0: a one-block launch after it)
        const bool fold = env_int("KVAD_HEAD_TAIL", 1) != 0;
        const GreedyTail tail{m->arrivals, m->token, m->pos, m->steps, out, m->out_cap, m->embed->precision,
                              m->embed->qs, m->embed->scales, m->embed->cols, m->x};
        rc = launch_gemv_argmax(ctx, head->precision, jobs[0].second, m->arg_v, m->arg_i, m->arg_n, ARGMAX_CAP,
                                fold ? &tail : nullptr);
        if (rc != KH_OK && rc != KH_DECLINED) return rc;
        if (rc == KH_OK && fold) return KH_OK;
        kept = rc == KH_OK;
    }
    if (!kept) {
        if ((rc = run_jobs(ctx, jobs))) return rc;
        hipLaunchKernelGGL(argmax_partial_kernel, dim3(ARGMAX_BLOCKS), dim3(256), 0, ctx->stream, m->logits,
                           (int)s.vocab, m->arg_v, m->arg_i);
        KH_HIP(hipGetLastError());
    }
    const NextEmbed ne{m->embed->precision, m->embed->qs, m->embed->scales, m->embed->cols, m->x};
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, ctx->stream, m->logits, (int)s.vocab, m->arg_v,
                       m->arg_i, kept ? m->arg_n : nullptr, m->token, m->pos, m->steps, out, m->out_cap, ne);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int ready(const kh_llm *m) {
    if (!m->embed || !m->final_norm || !m->rope_cos) return fail(KH_EINVAL, "llm: ends or rope tables not set");
    for (auto &L : m->layers)
        if (!L.q || !L.attn_norm) return fail(KH_EINVAL, "llm: a layer is not set");
    return KH_OK;
}

int check_weight_shape(const kh_weight *w, size_t rows, size_t cols, const char *what) {
    if (!w) return fail(KH_EINVAL, std::string("kh_llm_set_layer: ") + what + " is null");
    if (w->rows != rows || w->cols != cols)
        return fail(KH_EINVAL, std::string("kh_llm_set_layer: ") + what + " has the wrong shape");
    if (w->precision != KH_F32 && w->cols > 0x7fffffff) return fail(KH_EINVAL, "too wide");
    return KH_OK;
}

// ---- forward_each: n rows through the layers at once --------------------

// The rows' buffers, carved from one allocation for `cap` rows (base null:
// sizes only).  QActBatch codes take the widest activation of a block.
struct RowsBuf {
    float *x, *h, *q, *k, *v, *att, *g, *u, *logits, *pv;
    int *pi;
    int32_t *tok, *next;
    AttnRow *tab;  // [n_layer][n]: each row's cache and length
    QAct qa;
    void *ws;
    size_t ws_bytes, bytes;
};

// forward_each's buffers (pass = false), or a prompt pass's (pass = true):
// no per-row logits or argmax partials (the head reads the last row alone)
// and no attention workspace, which a pass sizes per launch (pass_ws).
RowsBuf rows_layout(const kh_llm_spec &s, size_t cap, char *base, bool pass = false) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        char *p = base ? base + off : nullptr;
        off += (bytes + 255) / 256 * 256;
        return p;
    };
    const size_t e = s.n_embd, qd = s.n_head * s.head_dim, kvd = s.n_kv_head * s.head_dim;
    const size_t wide = std::max(e, std::max(qd, s.n_ff)), nb = (cap * wide + BLOCK - 1) / BLOCK;
    RowsBuf b{};
    b.x = reinterpret_cast<float *>(take(4 * cap * e));
    b.h = reinterpret_cast<float *>(take(4 * cap * e));
    b.q = reinterpret_cast<float *>(take(4 * cap * qd));
    b.att = reinterpret_cast<float *>(take(4 * cap * qd));
    b.k = reinterpret_cast<float *>(take(4 * cap * kvd));
    b.v = reinterpret_cast<float *>(take(4 * cap * kvd));
    b.g = reinterpret_cast<float *>(take(4 * cap * s.n_ff));
    b.u = reinterpret_cast<float *>(take(4 * cap * s.n_ff));
    const size_t lr = pass ? 0 : cap;  // rows with logits of their own
    b.logits = reinterpret_cast<float *>(take(4 * lr * s.vocab));
    b.pv = reinterpret_cast<float *>(take(4 * lr * ARGMAX_BLOCKS));
    b.pi = reinterpret_cast<int *>(take(4 * lr * ARGMAX_BLOCKS));
    b.tok = reinterpret_cast<int32_t *>(take(4 * cap));
    b.next = reinterpret_cast<int32_t *>(take(4 * lr));
    b.tab = reinterpret_cast<AttnRow *>(take(sizeof(AttnRow) * cap * s.n_layer));
    b.qa.qs = reinterpret_cast<int8_t *>(take(cap * wide));
    b.qa.scales = reinterpret_cast<float *>(take(4 * nb));
    b.qa.sums = reinterpret_cast<int32_t *>(take(4 * nb));
    b.ws_bytes = pass ? 0 : attend_rows_ws_bytes((int)s.n_head, (int)s.head_dim, s.n_ctx, cap);
    b.ws = take(b.ws_bytes);
    b.bytes = off;
    return b;
}

// The captured passes name the weights, the tables and the rows' buffers:
// any change to those drops them.
void drop_rows_graphs(kh_llm *m) {
    for (auto &g : m->rows_graphs) (void)hipGraphExecDestroy(g.second);
    m->rows_graphs.clear();
    for (auto &g : m->pass_graphs) (void)hipGraphExecDestroy(g.second);
    m->pass_graphs.clear();
}

int ensure_rows(kh_llm *m, size_t n) {
    if (n <= m->rows_cap) return KH_OK;
    const size_t cap = (n + 7) / 8 * 8;
    KH_HIP(hipStreamSynchronize(m->ctx->stream));
    drop_rows_graphs(m);
    if (m->rows_buf) (void)hipFree(m->rows_buf);
    m->rows_buf = nullptr;
    m->rows_cap = 0;
    KH_HIP(hipMalloc(&m->rows_buf, rows_layout(m->spec, cap, nullptr).bytes));
    m->rows_cap = cap;
    return KH_OK;
}

// A prompt pass's rows (n of them) and its attention's partials for a launch
// of at most max_len positions; growing either drops the captured passes,
// which name the old buffers.
int ensure_pass(kh_llm *m, size_t n, size_t max_len) {
    kh_ctx *ctx = m->ctx;
    if (n > m->pass_cap) {
        const size_t cap = (n + 7) / 8 * 8;
        KH_HIP(hipStreamSynchronize(ctx->stream));
        drop_rows_graphs(m);
        if (m->pass_buf) (void)hipFree(m->pass_buf);
        m->pass_buf = nullptr;
        m->pass_cap = 0;
        KH_HIP(hipMalloc(&m->pass_buf, rows_layout(m->spec, cap, nullptr, true).bytes));
        m->pass_cap = cap;
    }
    const kh_llm_spec &s = m->spec;
    const size_t need = attend_rows_need_bytes(ctx, (int)s.n_head, (int)s.n_kv_head, (int)s.head_dim, max_len, n);
    if (need > m->pass_ws.bytes) {
        drop_rows_graphs(m);
        return ensure(ctx, m->pass_ws, need);
    }
    return KH_OK;
}

// y[n][rows] (+)= xs W^T (+bias): f32 weights on the f32 GEMM, quantised
// ones from the rows' codes in qa (matmul_bt, quant.rs:751; tensor.rs:102);
// with accumulate the product is added into y (the residual add).
// Projections of the same input (q/k/v, gate/up) take one multi-token GEMV
// launch up to this many rows (the weights stream once per launch; the GEMM
// would take a launch per weight, and at decode's small matrices its
// 128-row tiles leave most CUs idle).  A single projection (o, down, the
// head) follows kh_matmul's rule.
size_t rows_multi_max() {
    static const size_t v = (size_t)env_int("KVAD_ROWS_MULTI", 32);  // tuning knob
    return v;
}

int project(kh_ctx *ctx, const kh_weight *w, const float *xs, const QAct &qa, size_t n, const float *bias, float *y,
            int accumulate = 0) {
    if (w->precision == KH_F32) return launch_matmul(ctx, w, xs, n, bias, y, accumulate);
    if (n <= rows_multi_max() && matmul_takes_multi(n, w->rows, w->cols))
        return launch_gemv_multi_jobs(ctx, 1, &w, &bias, &y, &accumulate, qa, n);
    return launch_matmul_q(ctx, w, qa, n, bias, y, accumulate);
}

bool any_f32(std::initializer_list<const kh_weight *> ws) {
    for (auto w : ws)
        if (w->precision == KH_F32) return true;
    return false;
}

// Projections of the same input: one multi-token launch when they are all
// quantised alike and the rows are few, else one projection at a time.
int project_all(kh_ctx *ctx, int k, const kh_weight *const *w, const float *xs, const QAct &qa, size_t n,
                const float *const *bias, float *const *y) {
    bool one = n <= rows_multi_max();
    for (int i = 0; i < k; i++)
        one = one && w[i]->precision != KH_F32 && w[i]->precision == w[0]->precision && w[i]->cols == w[0]->cols;
    if (one) return launch_gemv_multi_jobs(ctx, k, w, bias, y, nullptr, qa, n);
    for (int i = 0; i < k; i++) {
        int rc = project(ctx, w[i], xs, qa, n, bias[i], y[i]);
        if (rc) return rc;
    }
    return KH_OK;
}

// rms_norm of the n rows, quantised for the projections that read it (and in
// f32 into h for the f32 ones).
int norm_rows(kh_ctx *ctx, const float *x, const float *w, size_t n, size_t e, float eps, bool need_f32, float *h,
              const QAct &qa) {
    if (e % BLOCK) return launch_rms_norm(ctx, x, w, n, e, eps, h);  // only f32 weights take such rows
    return launch_norm_qact(ctx, x, w, n, e, eps, need_f32 ? h : nullptr, qa);
}

// run_rows (llama.rs:224-289) over n rows whose table (tokens, and per layer
// each row's cache and length) is already on the device.
//   Rows::Each (batched decode): every row has a cache of its own; RoPE and
//   the cache push are fused into the attention's split kernel; then the
//   head over every row (llama.rs:412-416) and each row's greedy token.
//   Rows::Following (a prompt's pass, `following`): the rows are one
//   sequence's next positions in the held cache; every row is rotated and
//   pushed by a launch of its own before the attention, since row i attends
//   over the rows before it; then the head over the last row and its greedy
//   token (Transformer::head with all = false, llama.rs:404-411), which
//   becomes the session's next input.
// With a trace (the parity hook kh_debug_llm_trace_pass: a pass of the held
// sequence, never under capture) each sub-block's rows are copied out as it
// ends; len0 is the positions held before the pass.
int step_rows(kh_ctx *ctx, kh_llm *m, size_t n, const RowsBuf &b, size_t max_len, bool following = false,
              const kh_llm_trace *tr = nullptr, size_t len0 = 0) {
    const kh_llm_spec &s = m->spec;
    const size_t e = s.n_embd, qd = s.n_head * s.head_dim, kvd = s.n_kv_head * s.head_dim;
    const size_t qkvd = qd + 2 * kvd, held = len0 + n;
    int rc;
    if ((rc = launch_dequant_row_dev(ctx, m->embed, b.tok, b.x, n))) return rc;  // embed (llama.rs:384-391)
    if (tr && (rc = trace_copy(ctx, tr->x_embed, b.x, n * e))) return rc;
    for (size_t l = 0; l < s.n_layer; l++) {
        const kh_llm::Layer &L = m->layers[l];
        // ---- attention sub-block (llama.rs:241-275)
        if ((rc = norm_rows(ctx, b.x, L.attn_norm, n, e, s.eps, any_f32({L.q, L.k, L.v}), b.h, b.qa))) return rc;
        {
            const kh_weight *w[3] = {L.q, L.k, L.v};
            const float *bias[3] = {L.q_b, L.k_b, L.v_b};
            float *y[3] = {b.q, b.k, b.v};
            if ((rc = project_all(ctx, 3, w, b.h, b.qa, n, bias, y))) return rc;
        }
        if (tr && tr->qkv) {  // [n][q | k | v] per layer, before the rotation
            float *d = tr->qkv + l * n * qkvd;
            if ((rc = trace_rows(ctx, d, qkvd, b.q, qd, n)) || (rc = trace_rows(ctx, d + qd, qkvd, b.k, kvd, n)) ||
                (rc = trace_rows(ctx, d + qd + kvd, qkvd, b.v, kvd, n)))
                return rc;
        }
        // each row at its own position over its cache up to itself (run_rows,
        // llama.rs:249-271)
        const AttnRow *tab = b.tab + l * n;
        const AttnRope rp{b.k, b.v, m->rope_cos, m->rope_sin, L.q_norm, L.k_norm, s.eps, s.rope_interleaved, kvd};
        if (following && (rc = launch_rope_push_rows(ctx, (int)s.n_head, (int)s.n_kv_head, (int)s.head_dim, b.q,
                                                      b.k, b.v, tab, (int)n, kvd, kvd, rp)))
            return rc;
        if (following && attend_pass_fits((int)s.head_dim, kvd, kvd, max_len))
            rc = launch_attend_pass(ctx, (int)s.n_head, (int)s.n_kv_head, (int)s.head_dim, b.q, tab, (int)n, kvd, kvd,
                                    max_len, b.att);
        else
            rc = launch_attend_rows(ctx, (int)s.n_head, (int)s.n_kv_head, (int)s.head_dim, b.q, tab, (int)n, kvd, kvd,
                                    max_len, b.att, b.ws, b.ws_bytes, following ? nullptr : &rp);
        if (rc) return rc;
        if (tr && ((rc = trace_copy(ctx, tr->k_cache ? tr->k_cache + l * held * kvd : nullptr, m->kc[l], held * kvd)) ||
                   (rc = trace_copy(ctx, tr->v_cache ? tr->v_cache + l * held * kvd : nullptr, m->vc[l], held * kvd)) ||
                   (rc = trace_copy(ctx, tr->att ? tr->att + l * n * qd : nullptr, b.att, n * qd))))
            return rc;
        if (L.o->precision != KH_F32 && n <= (size_t)MULTI_TOKENS && n <= rows_multi_max() &&
            multi_stages_f32(L.o->precision, n, qd)) {
            // x += o(attn): the multi-token GEMV quantises the attention rows
            // itself, in its one launch, while they are narrow (past eight
            // rows it takes several, each quantising its rows in every
            // workgroup: measured slower than one quantisation launch at 32
            // rows)
            const float *no_bias = nullptr;
            const int acc = 1;
            if ((rc = launch_gemv_multi_jobs(ctx, 1, &L.o, &no_bias, &b.x, &acc, b.qa, n, b.att))) return rc;
        } else {
            if (L.o->precision != KH_F32 && (rc = launch_qact(ctx, b.att, n, qd, b.qa))) return rc;
            if ((rc = project(ctx, L.o, b.att, b.qa, n, nullptr, b.x, 1))) return rc;  // x += o(attn)
        }
        if (tr && (rc = trace_copy(ctx, tr->x_attn ? tr->x_attn + l * n * e : nullptr, b.x, n * e))) return rc;
        // ---- MLP sub-block (llama.rs:277-285, Ffn::run ffn.rs:370-375)
        if ((rc = norm_rows(ctx, b.x, L.mlp_norm, n, e, s.eps, any_f32({L.gate, L.up}), b.h, b.qa))) return rc;
        {
            const kh_weight *w[2] = {L.gate, L.up};
            const float *bias[2] = {nullptr, nullptr};
            float *y[2] = {b.g, b.u};
            if ((rc = project_all(ctx, 2, w, b.h, b.qa, n, bias, y))) return rc;
        }
        if (tr && ((rc = trace_copy(ctx, tr->gate ? tr->gate + l * n * s.n_ff : nullptr, b.g, n * s.n_ff)) ||
                   (rc = trace_copy(ctx, tr->up ? tr->up + l * n * s.n_ff : nullptr, b.u, n * s.n_ff))))
            return rc;
        if (L.down->precision != KH_F32) {  // QActBatch::new of swiglu(gate, up), then down
            if ((rc = launch_swiglu_qact(ctx, b.g, b.u, n, s.n_ff, b.qa))) return rc;
        } else if ((rc = launch_swiglu(ctx, b.g, b.u, n * s.n_ff))) {
            return rc;
        }
        if ((rc = project(ctx, L.down, b.g, b.qa, n, nullptr, b.x, 1))) return rc;  // x += mlp
        if (tr && (rc = trace_copy(ctx, tr->x_mlp ? tr->x_mlp + l * n * e : nullptr, b.x, n * e))) return rc;
    }
    if (following) return head_step(ctx, m, b.x + (n - 1) * e, false);
    // ---- head over every row (llama.rs:412-415), then each row's argmax
    const kh_weight *head = m->head ? m->head : m->embed;
    if ((rc = norm_rows(ctx, b.x, m->final_norm, n, e, s.eps, head->precision == KH_F32, b.h, b.qa))) return rc;
    if ((rc = project(ctx, head, b.h, b.qa, n, nullptr, b.logits))) return rc;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(ARGMAX_BLOCKS, (unsigned)n), dim3(256), 0, ctx->stream, b.logits,
                       (int)s.vocab, b.pv, b.pi);
    KH_HIP(hipGetLastError());
    hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)n), dim3(256), 0, ctx->stream, b.logits, (int)s.vocab,
                       b.pv, b.pi, b.next);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

// A cache of n_ctx positions per layer: a spare one if the session has it.
int take_cache(kh_llm *m, std::vector<float *> &k, std::vector<float *> &v) {
    if (!m->spare.empty()) {
        k = std::move(m->spare.back().first);
        v = std::move(m->spare.back().second);
        m->spare.pop_back();
        return KH_OK;
    }
    const size_t n = m->spec.n_ctx * m->spec.n_kv_head * m->spec.head_dim;
    k.assign(m->spec.n_layer, nullptr);
    v.assign(m->spec.n_layer, nullptr);
    int rc = KH_OK;
    for (size_t l = 0; l < m->spec.n_layer && !rc; l++)
        if ((rc = dev_alloc(&k[l], n)) == KH_OK) rc = dev_alloc(&v[l], n);
    if (rc) {
        for (float *p : k)
            if (p) (void)hipFree(p);
        for (float *p : v)
            if (p) (void)hipFree(p);
        k.clear();
        v.clear();
    }
    return rc;
}

// A cache no longer held: kept for the next park (a few), else freed.
void drop_cache(kh_llm *m, std::vector<float *> &k, std::vector<float *> &v) {
    if (m->spare.size() < 4) {
        m->spare.emplace_back(std::move(k), std::move(v));
    } else {
        (void)hipStreamSynchronize(m->ctx->stream);
        for (float *p : k) (void)hipFree(p);
        for (float *p : v) (void)hipFree(p);
    }
    k.clear();
    v.clear();
}

void drop_graph(kh_llm *m) {  // the captured steps name the held cache
    for (auto &g : m->graphs) (void)hipGraphExecDestroy(g.second);
    m->graphs.clear();
}

// The attention launch maximum for a step that ends with `len` positions
// held: the next power of two from 64 while that is at most attn_short (one
// split of the split kernel takes the whole sequence, no merge launch), else
// n_ctx.  Per-token calls and captured steps pick alike, so their results
// agree to the bit.
size_t bucket_max(const kh_llm *m, size_t len) {
    if (len > m->attn_short) return m->spec.n_ctx;
    size_t b = 64;
    while (b < len) b *= 2;
    return std::min(b, m->attn_short);
}

// Capture the step of bucket bm unless it is held (the launches read pos and
// token from the device, so one capture serves every step of the bucket).
int capture_step(kh_ctx *ctx, kh_llm *m, size_t bm) {
    if (m->graphs.count(bm)) return KH_OK;
    KH_HIP(hipStreamSynchronize(ctx->stream));
    m->attn_max = bm;
    hipGraph_t g = nullptr;
    KH_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    const int rc = step(ctx, m, nullptr, false);  // x: the previous step's argmax wrote it
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    m->graphs[bm] = x;
    return KH_OK;
}

// n steps from m->len: capture the buckets they cross first, then replay;
// the first step's input is the embedding row of the token held on the
// device (the captured steps take the row their argmax wrote).
int replay_steps(kh_ctx *ctx, kh_llm *m, size_t n) {
    int rc;
    for (size_t i = 0; i < n; i++)
        if ((rc = capture_step(ctx, m, bucket_max(m, m->len + i + 1)))) return rc;
    if ((rc = launch_dequant_row_dev(ctx, m->embed, m->token, m->x))) return rc;
    for (size_t i = 0; i < n; i++)
        KH_HIP(hipGraphLaunch(m->graphs.at(bucket_max(m, m->len + i + 1)), ctx->stream));
    return KH_OK;
}

// ---- a prompt read a pass at a time (Rows::Following) ---------------------

// Session::prefill_pass (model/mod.rs:866; CpuSession :1181-1183): whole
// chunks from the front, what is left over last.  The chunk is
// KVAD_PREFILL_CHUNK (the reference's knob, mod.rs:1004-1006) unless the
// caller set one (CpuSession::reading, :1079-1082), else DEFAULT_PASS: the
// reference's GPU backend reads 512 a pass (gpu/src/model.rs:892-897), and
// here a 640-token Qwen2.5-0.5B prompt takes 27 ms in passes of 64, 10 ms
// in passes of 256 and 6.4 ms in one pass (each pass is some 340 launches
// whatever its width, and wider passes give the GEMMs wider tiles).
constexpr size_t DEFAULT_PASS = 512;
size_t pass_len(const kh_llm *m, size_t left) {
    size_t c = m->chunk;
    if (!c) {
        const int v = env_int("KVAD_PREFILL_CHUNK", 0);
        c = v > 0 ? (size_t)v : DEFAULT_PASS;
    }
    c = std::min<size_t>(c, 65535);
    return std::min(left, c);
}

// The attention launch maximum of a pass ending with `held` positions: the
// next power of two from 64, at most n_ctx (a captured pass serves every
// pass of its row count up to that length).
size_t pass_bucket(const kh_llm *m, size_t held) {
    size_t b = 64;
    while (b < held) b *= 2;
    return std::min(b, m->spec.n_ctx);
}

// The table of a pass of n tokens: tokens, then per layer each row's cache
// (the held one) and its length after itself (positions len .. len + n - 1).
void pass_table(kh_llm *m, const int32_t *tokens, size_t n, size_t &tok_bytes, size_t &tab_bytes) {
    const kh_llm_spec &s = m->spec;
    tok_bytes = (4 * n + 15) & ~(size_t)15;
    tab_bytes = sizeof(AttnRow) * n * s.n_layer;
    m->rows_host.resize(tok_bytes + tab_bytes);
    std::copy(tokens, tokens + n, reinterpret_cast<int32_t *>(m->rows_host.data()));
    AttnRow *tab = reinterpret_cast<AttnRow *>(m->rows_host.data() + tok_bytes);
    for (size_t l = 0; l < s.n_layer; l++)
        for (size_t i = 0; i < n; i++) tab[l * n + i] = AttnRow{m->kc[l], m->vc[l], (int)(m->len + i + 1)};
}

// One pass of n >= 1 tokens of the held sequence: n == 1 is the one-token
// step; more rows run step_rows(following), captured per (n, bucket), or
// eagerly with a trace.  The state afterwards is the step's: the greedy next
// token is the input, the position is len + n.  Returns with the stream
// synchronised (the table's host copy is reused by the next pass).
int run_pass(kh_ctx *ctx, kh_llm *m, const int32_t *tokens, size_t n, const kh_llm_trace *tr = nullptr) {
    int rc;
    if (n == 1 && !tr) {
        const int32_t st[3] = {tokens[0], (int32_t)m->len, 0};
        KH_HIP(hipMemcpyAsync(m->state, st, sizeof st, hipMemcpyHostToDevice, ctx->stream));
        m->attn_max = bucket_max(m, m->len + 1);
        if ((rc = step(ctx, m))) return rc;
        KH_HIP(hipStreamSynchronize(ctx->stream));
        m->len += 1;
        return KH_OK;
    }
    const size_t bm = pass_bucket(m, m->len + n);
    if ((rc = ensure_pass(m, n, bm))) return rc;
    RowsBuf b = rows_layout(m->spec, m->pass_cap, static_cast<char *>(m->pass_buf), true);
    b.ws = m->pass_ws.ptr;
    b.ws_bytes = m->pass_ws.bytes;
    size_t tok_bytes, tab_bytes;
    pass_table(m, tokens, n, tok_bytes, tab_bytes);
    // the head's tail advances the position past the last row
    const int32_t st[3] = {tokens[n - 1], (int32_t)(m->len + n - 1), 0};
    KH_HIP(hipMemcpyAsync(m->state, st, sizeof st, hipMemcpyHostToDevice, ctx->stream));
    KH_HIP(hipMemcpyAsync(b.tok, m->rows_host.data(), tok_bytes, hipMemcpyHostToDevice, ctx->stream));
    KH_HIP(hipMemcpyAsync(b.tab, m->rows_host.data() + tok_bytes, tab_bytes, hipMemcpyHostToDevice, ctx->stream));
    if (tr) {
        if ((rc = step_rows(ctx, m, n, b, bm, true, tr, m->len))) return rc;
    } else {
        const std::pair<size_t, size_t> key{n, bm};
        auto it = m->pass_graphs.find(key);
        if (it == m->pass_graphs.end()) {
            if ((rc = gemm_split_reserve(ctx))) return rc;
            KH_HIP(hipStreamSynchronize(ctx->stream));
            hipGraph_t g = nullptr;
            KH_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
            rc = step_rows(ctx, m, n, b, bm, true);
            hipError_t e = hipStreamEndCapture(ctx->stream, &g);
            if (rc) {
                if (g) (void)hipGraphDestroy(g);
                return rc;
            }
            if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
            hipGraphExec_t x = nullptr;
            e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
            it = m->pass_graphs.emplace(key, x).first;
        }
        KH_HIP(hipGraphLaunch(it->second, ctx->stream));
    }
    KH_HIP(hipStreamSynchronize(ctx->stream));
    m->len += n;
    return KH_OK;
}

// Tokens of the held sequence, checked against the vocabulary and the window.
int check_tokens(const kh_llm *m, const int32_t *tokens, size_t n, const char *what) {
    for (size_t i = 0; i < n; i++)
        if (tokens[i] < 0 || (size_t)tokens[i] >= m->spec.vocab)
            return fail(KH_EINVAL, std::string(what) + ": token out of range");
    if (m->len + n > m->spec.n_ctx)
        return fail(KH_EINVAL, std::string(what) + ": the tokens would overrun the context window");
    return KH_OK;
}

}  // namespace
}  // namespace kh

using namespace kh;

extern "C" {

int kh_llm_new(kh_ctx *ctx, const kh_llm_spec *spec, kh_llm **out) {
    if (!ctx || !spec || !out) return fail(KH_EINVAL, "kh_llm_new: null argument");
    *out = nullptr;
    const kh_llm_spec &s = *spec;
    if (!s.n_layer || !s.n_embd || !s.n_head || !s.n_kv_head || !s.head_dim || !s.n_ff || !s.vocab || !s.n_ctx ||
        s.n_head % s.n_kv_head)
        return fail(KH_EINVAL, "kh_llm_new: every size must be positive and n_kv_head divide n_head");
    if ((s.head_dim != 64 && s.head_dim != 128) || s.n_ctx > (1u << 20) || s.n_head + s.n_kv_head + 1 > 65535)
        return fail(KH_DECLINED, "kh_llm_new: head_dim 64 or 128 and a context up to 2^20 positions");
    if (s.n_ff % BLOCK || s.n_embd % 4) return fail(KH_EINVAL, "kh_llm_new: n_ff % 32 and n_embd % 4 must be 0");
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    std::unique_ptr<kh_llm> m(new kh_llm());
    m->ctx = ctx;
    m->spec = s;
    m->layers.assign(s.n_layer, kh_llm::Layer{});
    const size_t kvd = s.n_kv_head * s.head_dim, qd = s.n_head * s.head_dim;
    int rc;
    m->kc.assign(s.n_layer, nullptr);
    m->vc.assign(s.n_layer, nullptr);
    for (size_t l = 0; l < s.n_layer; l++) {
        if ((rc = dev_alloc(&m->kc[l], s.n_ctx * kvd)) || (rc = dev_alloc(&m->vc[l], s.n_ctx * kvd))) return rc;
    }
    // codes of the widest activation quantised ahead of its GEMV
    const size_t hq_n = std::max(s.n_ff, std::max(qd, s.n_embd));
    if ((rc = dev_alloc(&m->x, s.n_embd)) || (rc = dev_alloc(&m->h, s.n_embd)) ||
        (rc = dev_alloc(&m->qkv, qd + 2 * kvd)) || (rc = dev_alloc(&m->att, qd)) || (rc = dev_alloc(&m->g, s.n_ff)) ||
        (rc = dev_alloc(&m->u, s.n_ff)) || (rc = dev_alloc(&m->hsw, s.n_ff)) || (rc = dev_alloc(&m->logits, s.vocab)) ||
        (rc = dev_alloc(&m->hq.qs, hq_n)) || (rc = dev_alloc(&m->hq.scales, hq_n / BLOCK)) ||
        (rc = dev_alloc(&m->hq.sums, hq_n / BLOCK)) || (rc = dev_alloc(&m->state, 3)) ||
        (rc = dev_alloc(&m->arg_v, ARGMAX_CAP)) || (rc = dev_alloc(&m->arg_i, ARGMAX_CAP)) ||
        (rc = dev_alloc(&m->arg_n, 1)) || (rc = dev_alloc(&m->arrivals, 1)))
        return rc;
    m->token = m->state, m->pos = m->state + 1, m->steps = m->state + 2;
    KH_HIP(hipMemset(m->state, 0, 3 * sizeof(int32_t)));
    KH_HIP(hipMemset(m->arrivals, 0, sizeof(unsigned)));
    m->attn_ws_bytes = attend_ws_bytes((int)s.n_head, (int)s.n_kv_head, (int)s.head_dim, s.n_ctx);
    m->attn_short = std::min(attend_single_max((int)s.head_dim), s.n_ctx);
    m->attn_max = s.n_ctx;
    KH_HIP(hipMalloc(&m->attn_ws, m->attn_ws_bytes));
    *out = m.release();
    return KH_OK;
}

int kh_llm_free(kh_llm *m) {
    if (!m) return KH_OK;
    {
        std::lock_guard<std::recursive_mutex> lock(m->ctx->mu);
        (void)hipSetDevice(m->ctx->device);
        (void)hipStreamSynchronize(m->ctx->stream);
        drop_graph(m);
        drop_rows_graphs(m);
        for (auto p : m->kc) (void)hipFree(p);
        for (auto p : m->vc) (void)hipFree(p);
        for (auto &c : m->spare) {
            for (auto p : c.first) (void)hipFree(p);
            for (auto p : c.second) (void)hipFree(p);
        }
        for (kh_llm_parked *p : m->parked) p->owner = nullptr;  // theirs now, freed with the handle
        if (m->rows_buf) (void)hipFree(m->rows_buf);
        if (m->pass_buf) (void)hipFree(m->pass_buf);
        if (m->pass_ws.ptr) (void)hipFree(m->pass_ws.ptr);
        for (auto &L : m->layers)
            for (float *p : {L.attn_norm, L.mlp_norm, L.q_b, L.k_b, L.v_b, L.q_norm, L.k_norm})
                if (p) (void)hipFree(p);
        for (void *p : {(void *)m->x, (void *)m->h, (void *)m->qkv, (void *)m->att, (void *)m->g, (void *)m->u,
                        (void *)m->hsw,
                        (void *)m->logits, (void *)m->hq.qs, (void *)m->hq.scales, (void *)m->hq.sums,
                        (void *)m->state, (void *)m->final_norm, (void *)m->rope_cos, (void *)m->rope_sin,
                        m->attn_ws, (void *)m->out, (void *)m->arg_v, (void *)m->arg_i, (void *)m->arg_n, (void *)m->arrivals})
            if (p) (void)hipFree(p);
    }
    delete m;
    return KH_OK;
}

int kh_llm_set_layer(kh_llm *m, size_t l, const kh_weight *q, const kh_weight *k, const kh_weight *v,
                     const kh_weight *o, const kh_weight *gate, const kh_weight *up, const kh_weight *down,
                     const float *attn_norm, const float *mlp_norm, const float *q_b, const float *k_b,
                     const float *v_b, const float *q_norm, const float *k_norm) {
    if (!m || !attn_norm || !mlp_norm) return fail(KH_EINVAL, "kh_llm_set_layer: null argument");
    const kh_llm_spec &s = m->spec;
    if (l >= s.n_layer) return fail(KH_EINVAL, "kh_llm_set_layer: no such layer");
    const size_t qd = s.n_head * s.head_dim, kvd = s.n_kv_head * s.head_dim;
    int rc;
    if ((rc = check_weight_shape(q, qd, s.n_embd, "q")) || (rc = check_weight_shape(k, kvd, s.n_embd, "k")) ||
        (rc = check_weight_shape(v, kvd, s.n_embd, "v")) || (rc = check_weight_shape(o, s.n_embd, qd, "o")) ||
        (rc = check_weight_shape(gate, s.n_ff, s.n_embd, "gate")) ||
        (rc = check_weight_shape(up, s.n_ff, s.n_embd, "up")) ||
        (rc = check_weight_shape(down, s.n_embd, s.n_ff, "down")))
        return rc;
    std::lock_guard<std::recursive_mutex> lock(m->ctx->mu);
    (void)hipSetDevice(m->ctx->device);
    kh_llm::Layer &L = m->layers[l];
    for (float *p : {L.attn_norm, L.mlp_norm, L.q_b, L.k_b, L.v_b, L.q_norm, L.k_norm})
        if (p) (void)hipFree(p);
    L = kh_llm::Layer{};
    L.q = q, L.k = k, L.v = v, L.o = o, L.gate = gate, L.up = up, L.down = down;
    if ((rc = dev_vector(&L.attn_norm, attn_norm, s.n_embd)) || (rc = dev_vector(&L.mlp_norm, mlp_norm, s.n_embd)) ||
        (rc = dev_vector(&L.q_b, q_b, qd)) || (rc = dev_vector(&L.k_b, k_b, kvd)) ||
        (rc = dev_vector(&L.v_b, v_b, kvd)) || (rc = dev_vector(&L.q_norm, q_norm, s.head_dim)) ||
        (rc = dev_vector(&L.k_norm, k_norm, s.head_dim)))
        return rc;
    drop_graph(m);
    drop_rows_graphs(m);
    return KH_OK;
}

int kh_llm_set_ends(kh_llm *m, const kh_weight *embed, const float *final_norm, const kh_weight *lm_head) {
    if (!m || !embed || !final_norm) return fail(KH_EINVAL, "kh_llm_set_ends: null argument");
    const kh_llm_spec &s = m->spec;
    if (embed->rows != s.vocab || embed->cols != s.n_embd)
        return fail(KH_EINVAL, "kh_llm_set_ends: the embedding is [vocab, n_embd]");
    if (lm_head && (lm_head->rows != s.vocab || lm_head->cols != s.n_embd))
        return fail(KH_EINVAL, "kh_llm_set_ends: the head is [vocab, n_embd]");
    std::lock_guard<std::recursive_mutex> lock(m->ctx->mu);
    (void)hipSetDevice(m->ctx->device);
    if (m->final_norm) (void)hipFree(m->final_norm);
    int rc = dev_vector(&m->final_norm, final_norm, s.n_embd);
    if (rc) return rc;
    m->embed = embed;
    m->head = lm_head;
    drop_graph(m);
    drop_rows_graphs(m);
    return KH_OK;
}

int kh_llm_set_rope(kh_llm *m, const float *cos_t, const float *sin_t, size_t max_pos) {
    if (!m || !cos_t || !sin_t) return fail(KH_EINVAL, "kh_llm_set_rope: null argument");
    if (max_pos < m->spec.n_ctx) return fail(KH_EINVAL, "kh_llm_set_rope: the tables must cover n_ctx positions");
    std::lock_guard<std::recursive_mutex> lock(m->ctx->mu);
    (void)hipSetDevice(m->ctx->device);
    const size_t n = m->spec.n_ctx * (m->spec.head_dim / 2);
    if (m->rope_cos) (void)hipFree(m->rope_cos);
    if (m->rope_sin) (void)hipFree(m->rope_sin);
    m->rope_cos = m->rope_sin = nullptr;
    drop_graph(m);  // the captured passes name the old tables
    drop_rows_graphs(m);
    int rc;
    if ((rc = dev_vector(&m->rope_cos, cos_t, n)) || (rc = dev_vector(&m->rope_sin, sin_t, n))) return rc;
    return KH_OK;
}

int kh_llm_len(const kh_llm *m, size_t *len) {
    if (!m || !len) return fail(KH_EINVAL, "kh_llm_len: null argument");
    *len = m->len;
    return KH_OK;
}

int kh_llm_truncate(kh_llm *m, size_t len) {
    if (!m) return fail(KH_EINVAL, "kh_llm_truncate: null argument");
    std::lock_guard<std::recursive_mutex> lock(m->ctx->mu);
    (void)hipSetDevice(m->ctx->device);
    if (len < m->len) m->len = len;  // KvCache::truncate keeps a prefix, never extends (mod.rs:709-725)
    const int32_t p = (int32_t)m->len;
    KH_HIP(hipMemcpyAsync(m->pos, &p, 4, hipMemcpyHostToDevice, m->ctx->stream));
    KH_HIP(hipStreamSynchronize(m->ctx->stream));
    return KH_OK;
}

int kh_llm_forward(kh_ctx *ctx, kh_llm *m, int32_t token, float *logits, int32_t *next) {
    if (!ctx || !m || m->ctx != ctx) return fail(KH_EINVAL, "kh_llm_forward: null argument or foreign context");
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    int rc = ready(m);
    if (rc) return rc;
    if (token < 0 || (size_t)token >= m->spec.vocab) return fail(KH_EINVAL, "kh_llm_forward: token out of range");
    if (m->len >= m->spec.n_ctx) return fail(KH_EINVAL, "kh_llm_forward: the context window is full");
    const int32_t st[3] = {token, (int32_t)m->len, 0};
    KH_HIP(hipMemcpyAsync(m->state, st, sizeof st, hipMemcpyHostToDevice, ctx->stream));
    m->attn_max = bucket_max(m, m->len + 1);
    if ((rc = step(ctx, m))) return rc;
    if (logits) KH_HIP(hipMemcpyAsync(logits, m->logits, 4 * m->spec.vocab, hipMemcpyDeviceToHost, ctx->stream));
    int32_t nt = 0;
    KH_HIP(hipMemcpyAsync(&nt, m->token, 4, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    m->len += 1;
    if (next) *next = nt;
    return KH_OK;
}

int kh_llm_forward_tokens(kh_ctx *ctx, kh_llm *m, const int32_t *tokens, size_t n, float *logits, int32_t *next) {
    if (!ctx || !m || m->ctx != ctx) return fail(KH_EINVAL, "kh_llm_forward_tokens: null argument or foreign context");
    if (n == 0) return KH_OK;
    if (!tokens) return fail(KH_EINVAL, "kh_llm_forward_tokens: null tokens");
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    int rc = ready(m);
    if (rc || (rc = check_tokens(m, tokens, n, "kh_llm_forward_tokens"))) return rc;
    // Session::forward (CpuSession, mod.rs:1149-1158): the tokens in passes
    // cut where prefill_pass says, the last pass's logits returned
    for (size_t at = 0; at < n;) {
        const size_t pass = pass_len(m, n - at);
        if ((rc = run_pass(ctx, m, tokens + at, pass))) return rc;
        at += pass;
    }
    if (logits) KH_HIP(hipMemcpyAsync(logits, m->logits, 4 * m->spec.vocab, hipMemcpyDeviceToHost, ctx->stream));
    int32_t nt = 0;
    KH_HIP(hipMemcpyAsync(&nt, m->token, 4, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    if (next) *next = nt;
    return KH_OK;
}

int kh_llm_prefill_pass(const kh_llm *m, size_t left, size_t *pass) {
    if (!m || !pass) return fail(KH_EINVAL, "kh_llm_prefill_pass: null argument");
    *pass = pass_len(m, left);
    return KH_OK;
}

int kh_llm_set_prefill_chunk(kh_llm *m, size_t chunk) {
    if (!m) return fail(KH_EINVAL, "kh_llm_set_prefill_chunk: null argument");
    if (chunk > 65535) return fail(KH_EINVAL, "kh_llm_set_prefill_chunk: at most 65535 tokens a pass");
    std::lock_guard<std::recursive_mutex> lock(m->ctx->mu);
    m->chunk = chunk;  // 0: KVAD_PREFILL_CHUNK, else 64
    return KH_OK;
}

int kh_debug_llm_trace_pass(kh_ctx *ctx, kh_llm *m, const int32_t *tokens, size_t n, const kh_llm_trace *tr) {
    if (!ctx || !m || m->ctx != ctx || !tr || !tokens || n == 0)
        return fail(KH_EINVAL, "kh_debug_llm_trace_pass: null argument or no tokens");
    if (n > 65535) return fail(KH_EINVAL, "kh_debug_llm_trace_pass: at most 65535 tokens a pass");
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    int rc = ready(m);
    if (rc || (rc = check_tokens(m, tokens, n, "kh_debug_llm_trace_pass"))) return rc;
    if ((rc = run_pass(ctx, m, tokens, n, tr))) return rc;
    if (tr->logits) KH_HIP(hipMemcpyAsync(tr->logits, m->logits, 4 * m->spec.vocab, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

int kh_debug_llm_trace(kh_ctx *ctx, kh_llm *m, int32_t token, const kh_llm_trace *tr) {
    if (!ctx || !m || m->ctx != ctx || !tr) return fail(KH_EINVAL, "kh_debug_llm_trace: null argument");
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    int rc = ready(m);
    if (rc) return rc;
    if (token < 0 || (size_t)token >= m->spec.vocab) return fail(KH_EINVAL, "kh_debug_llm_trace: token out of range");
    if (m->len >= m->spec.n_ctx) return fail(KH_EINVAL, "kh_debug_llm_trace: the context window is full");
    const int32_t st[3] = {token, (int32_t)m->len, 0};
    KH_HIP(hipMemcpyAsync(m->state, st, sizeof st, hipMemcpyHostToDevice, ctx->stream));
    m->attn_max = bucket_max(m, m->len + 1);
    if ((rc = step(ctx, m, tr))) return rc;
    if (tr->logits) KH_HIP(hipMemcpyAsync(tr->logits, m->logits, 4 * m->spec.vocab, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    m->len += 1;
    return KH_OK;
}

int kh_llm_generate(kh_ctx *ctx, kh_llm *m, int32_t token, size_t n, int32_t *tokens) {
    if (!ctx || !m || m->ctx != ctx || (n && !tokens)) return fail(KH_EINVAL, "kh_llm_generate: null argument");
    if (n == 0) return KH_OK;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    int rc = ready(m);
    if (rc) return rc;
    if (token < 0 || (size_t)token >= m->spec.vocab) return fail(KH_EINVAL, "kh_llm_generate: token out of range");
    if (m->len + n > m->spec.n_ctx) return fail(KH_EINVAL, "kh_llm_generate: the steps would overrun the context");
    if (m->out_cap < n) {  // the record of generated tokens
        if (m->out) {
            KH_HIP(hipStreamSynchronize(ctx->stream));
            (void)hipFree(m->out);
            m->out = nullptr;
        }
        drop_graph(m);
        KH_HIP(hipMalloc(reinterpret_cast<void **>(&m->out), 4 * n));
        m->out_cap = (int)n;
    }
    const int32_t st[3] = {token, (int32_t)m->len, 0};
    KH_HIP(hipMemcpyAsync(m->state, st, sizeof st, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = replay_steps(ctx, m, n))) return rc;
    KH_HIP(hipMemcpyAsync(tokens, m->out, 4 * n, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    m->len += n;
    return KH_OK;
}

int kh_llm_generate_launch(kh_ctx *ctx, kh_llm *m, size_t n) {
    // Replays n more steps of an already-captured graph from the device state
    // as it stands, without copying anything back (for timing).
    if (!ctx || !m || m->graphs.empty())
        return fail(KH_EINVAL, "kh_llm_generate_launch: no captured step");
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    if (m->len + n > m->spec.n_ctx) return fail(KH_EINVAL, "kh_llm_generate_launch: the steps would overrun the context");
    const int rc = replay_steps(ctx, m, n);
    if (rc) return rc;
    m->len += n;
    return KH_OK;
}

int kh_llm_park(kh_llm *m, kh_llm_parked **out) {
    if (!m || !out) return fail(KH_EINVAL, "kh_llm_park: null argument");
    *out = nullptr;
    std::lock_guard<std::recursive_mutex> lock(m->ctx->mu);
    (void)hipSetDevice(m->ctx->device);
    std::vector<float *> k, v;
    int rc = take_cache(m, k, v);  // the empty one left in its place
    if (rc) return rc;
    std::unique_ptr<kh_llm_parked> p(new kh_llm_parked());
    p->owner = m;
    p->device = m->ctx->device;
    p->k = std::move(m->kc);
    p->v = std::move(m->vc);
    p->len = m->len;
    m->kc = std::move(k);
    m->vc = std::move(v);
    m->len = 0;
    drop_graph(m);
    const int32_t st[3] = {0, 0, 0};
    KH_HIP(hipMemcpyAsync(m->state, st, sizeof st, hipMemcpyHostToDevice, m->ctx->stream));
    KH_HIP(hipStreamSynchronize(m->ctx->stream));
    m->parked.insert(p.get());
    *out = p.release();
    return KH_OK;
}

int kh_llm_parked_free(kh_llm_parked *p) {
    if (!p) return KH_OK;
    if (kh_llm *m = p->owner) {
        std::lock_guard<std::recursive_mutex> lock(m->ctx->mu);
        (void)hipSetDevice(m->ctx->device);
        m->parked.erase(p);
        drop_cache(m, p->k, p->v);
    } else {  // the session is gone: the cache is this handle's alone
        (void)hipSetDevice(p->device);
        (void)hipDeviceSynchronize();
        for (float *q : p->k) (void)hipFree(q);
        for (float *q : p->v) (void)hipFree(q);
    }
    delete p;
    return KH_OK;
}

int kh_llm_resume(kh_llm *m, kh_llm_parked *p) {
    if (!m || !p) return fail(KH_EINVAL, "kh_llm_resume: null argument");
    if (p->owner != m) {
        kh_llm_parked_free(p);
        return fail(KH_EINVAL, "kh_llm_resume: that cache was not this backend's");
    }
    std::lock_guard<std::recursive_mutex> lock(m->ctx->mu);
    (void)hipSetDevice(m->ctx->device);
    // the swap is host-side, so the handle is consumed whatever follows; a
    // dropped cache is reused only by later work on the same stream
    m->parked.erase(p);
    drop_cache(m, m->kc, m->vc);  // the conversation held until now is dropped
    m->kc = std::move(p->k);
    m->vc = std::move(p->v);
    m->len = p->len;
    delete p;
    drop_graph(m);
    const int32_t st[3] = {0, (int32_t)m->len, 0};
    KH_HIP(hipMemcpyAsync(m->state, st, sizeof st, hipMemcpyHostToDevice, m->ctx->stream));
    KH_HIP(hipStreamSynchronize(m->ctx->stream));
    return KH_OK;
}

int kh_llm_parked_len(const kh_llm_parked *p, size_t *len) {
    if (!p || !len) return fail(KH_EINVAL, "kh_llm_parked_len: null argument");
    *len = p->len;
    return KH_OK;
}

int kh_llm_forward_each(kh_ctx *ctx, kh_llm *m, size_t n, const int32_t *tokens, kh_llm_parked *const *caches,
                        float *logits, int32_t *next) {
    if (!ctx || !m || m->ctx != ctx) return fail(KH_EINVAL, "kh_llm_forward_each: null argument or foreign context");
    if (n == 0) return KH_OK;
    if (!tokens || !caches) return fail(KH_EINVAL, "kh_llm_forward_each: null argument");
    const kh_llm_spec &s = m->spec;
    if (n > 65535) return fail(KH_EINVAL, "kh_llm_forward_each: at most 65535 conversations at once");
    std::set<const kh_llm_parked *> seen;
    for (size_t i = 0; i < n; i++) {
        const kh_llm_parked *p = caches[i];
        if (!p) return fail(KH_EINVAL, "kh_llm_forward_each: null cache");
        if (p->owner != m) return fail(KH_EINVAL, "kh_llm_forward_each: that cache was not this backend's");
        if (!seen.insert(p).second) return fail(KH_EINVAL, "kh_llm_forward_each: a conversation given twice");
        if (tokens[i] < 0 || (size_t)tokens[i] >= s.vocab)
            return fail(KH_EINVAL, "kh_llm_forward_each: token out of range");
        if (p->len >= s.n_ctx) return fail(KH_EINVAL, "kh_llm_forward_each: a context window is full");
    }
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    int rc = ready(m);
    if (rc) return rc;
    if ((rc = ensure_rows(m, n))) return rc;
    const RowsBuf b = rows_layout(s, m->rows_cap, static_cast<char *>(m->rows_buf));
    // the table: tokens, then per layer each row's cache and its length
    // after this token (positions are fixed before anything is pushed,
    // llama.rs:229-236)
    const size_t tok_bytes = (4 * n + 15) & ~(size_t)15, tab_bytes = sizeof(AttnRow) * n * s.n_layer;
    m->rows_host.resize(tok_bytes + tab_bytes);
    std::copy(tokens, tokens + n, reinterpret_cast<int32_t *>(m->rows_host.data()));
    AttnRow *tab = reinterpret_cast<AttnRow *>(m->rows_host.data() + tok_bytes);
    size_t longest = 0;
    for (size_t i = 0; i < n; i++) longest = std::max(longest, caches[i]->len + 1);
    for (size_t l = 0; l < s.n_layer; l++)
        for (size_t i = 0; i < n; i++) tab[l * n + i] = AttnRow{caches[i]->k[l], caches[i]->v[l], (int)caches[i]->len + 1};
    // the pass for n rows reads everything it varies on from the table, so
    // it is captured once per n and attention bucket (of the longest row) and replayed
    const size_t bm = bucket_max(m, longest);
    const std::pair<size_t, size_t> key{n, bm};
    auto it = m->rows_graphs.find(key);
    if (it == m->rows_graphs.end()) {
        if ((rc = gemm_split_reserve(ctx))) return rc;
        KH_HIP(hipStreamSynchronize(ctx->stream));
        hipGraph_t g = nullptr;
        KH_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
        rc = step_rows(ctx, m, n, b, bm);
        hipError_t e = hipStreamEndCapture(ctx->stream, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
        hipGraphExec_t x = nullptr;
        e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
        it = m->rows_graphs.emplace(key, x).first;
    }
    KH_HIP(hipMemcpyAsync(b.tok, m->rows_host.data(), tok_bytes, hipMemcpyHostToDevice, ctx->stream));
    KH_HIP(hipMemcpyAsync(b.tab, tab, tab_bytes, hipMemcpyHostToDevice, ctx->stream));
    KH_HIP(hipGraphLaunch(it->second, ctx->stream));
    if (logits) KH_HIP(hipMemcpyAsync(logits, b.logits, 4 * n * s.vocab, hipMemcpyDeviceToHost, ctx->stream));
    if (next) KH_HIP(hipMemcpyAsync(next, b.next, 4 * n, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    for (size_t i = 0; i < n; i++) caches[i]->len += 1;  // Rows::advance (llama.rs:322-326)
    return KH_OK;
}

}  // extern "C"
