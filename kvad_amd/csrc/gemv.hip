// Single-token GEMV for kvad's q8 / q4 layouts, GGML Q4_K blocks and f32
// weights, plus the activation quantiser.
//
// Reference: Weight::matvec_bt / qrow (crates/llm/src/quant.rs:410-512),
// q4_row_dots (quant.rs:168-189), matvec_many (quant.rs:628-671),
// QActivation::new (quant.rs:1044-1066), tensor::matvec_bt (tensor.rs:56-79),
// Q4_K decoding (crates/gpu/src/mpp.rs:241-315).
//
// Shape of the kernel.  A workgroup (8 waves) first stages the activation in
// LDS as int8 codes, per-32 scales and code sums -- quantising the f32 input
// itself (QActivation::new, fused into the GEMV so a matvec is one launch),
// or copying codes a producer already made.  Each wave then owns R weight
// rows at a time.  A row is cut into 16-byte chunks (q8: half a 32-block;
// q4: one block; Q4_K: half of two sub-blocks' nibbles) and lane l takes
// chunks l, l+64, l+128, ... so one load instruction of the wave moves 1 KiB
// of contiguous weight bytes.  Weight loads are buffer loads: a read past the
// end of an array returns zeros, so tails need no branches (a chunk past the
// row end meets zero activations, a row past the last meets zero weights).
// Block dots are v_dot4 on int8 lanes; a 32-block split over two lanes is
// joined with a DPP lane swap, so every i32 is exact.  The scaled f32 terms
// are summed per lane in chunk order, then across the wave with DPP.
//
// Bit-exactness.  Activation codes and block dots equal the reference's
// integers.  Each f32 term uses the reference's operation order (quant.rs:449:
// (ws * xs) * d), with contraction off.  The sum over blocks is a wave tree,
// so outputs agree to rounding (1e-5 relative), not to the bit.  The per-lane
// order depends only on the chunk index, never on the unroll (CPL) or the
// rows per wave (R), so a row computed in a matvec_many launch equals the
// same row computed alone, to the bit.
#include "gemv_core.hpp"
#include "route.hpp"

#include <vector>

namespace kh {
namespace {


__global__ __launch_bounds__(256) void qact_kernel(const float *__restrict__ x, size_t nblocks,
                                                  int8_t *__restrict__ qs, float *__restrict__ scales,
                                                  int32_t *__restrict__ sums) {
    size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t b = tid >> 3;
    int sub = threadIdx.x & 7;
    bool ok = b < nblocks;
    float4 v = ok ? reinterpret_cast<const float4 *>(x)[b * 8 + sub] : make_float4(0.f, 0.f, 0.f, 0.f);
    float scale;
    int s;
    int packed = quantize4(v, &scale, &s);
    if (ok) {
        reinterpret_cast<int *>(qs)[b * 8 + sub] = packed;
        if (sub == 0) {
            scales[b] = scale;
            sums[b] = s;
        }
    }
}

// The activation quantiser's arithmetic against its definition for every
// float: counts[0] scales and counts[1] inverses (qscale of each finite
// amax >= 0) that differ from the IEEE quotients amax / 127 and 1 / scale,
// counts[2] codes (qround of each of the 2^32 patterns) that differ from
// Rust's t.round().clamp(-127.0, 127.0) as i8 (NaN to 0).
__global__ __launch_bounds__(256) void quant_check_kernel(unsigned long long *counts) {
    unsigned long long ns = 0, ni = 0, nr = 0;
    const unsigned long long stride = (unsigned long long)gridDim.x * blockDim.x;
    for (unsigned long long u = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; u < (1ull << 32);
         u += stride) {
        const unsigned b = (unsigned)u;
        if (b <= 0x7f7fffffu) {
            const float a = __builtin_bit_cast(float, b);
            const float sref = a / 127.0f;
            const float iref = sref > 0.0f ? 1.0f / sref : 0.0f;
            float sc, inv;
            qscale(a, sc, inv);
            ns += __builtin_bit_cast(unsigned, sc) != __builtin_bit_cast(unsigned, sref);
            ni += __builtin_bit_cast(unsigned, inv) != __builtin_bit_cast(unsigned, iref);
        }
        const float t = __builtin_bit_cast(float, b);
        int ref = 0;
        if (t == t) ref = (int)fminf(fmaxf(roundf(t), -127.0f), 127.0f);
        nr += qround(t) != ref;
    }
    if (ns) atomicAdd(counts + 0, ns);
    if (ni) atomicAdd(counts + 1, ni);
    if (nr) atomicAdd(counts + 2, nr);
}

// QActBatch::new of h = swiglu(g, u) (tensor.rs:344-350, quant.rs:693-714).
__global__ __launch_bounds__(256) void swiglu_qact_kernel(const float *__restrict__ g, const float *__restrict__ u,
                                                         size_t nblocks, int8_t *__restrict__ qs,
                                                         float *__restrict__ scales, int32_t *__restrict__ sums) {
    size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t b = tid >> 3;
    int sub = threadIdx.x & 7;
    bool ok = b < nblocks;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (ok) {
        const float4 a = reinterpret_cast<const float4 *>(g)[b * 8 + sub];
        const float4 c = reinterpret_cast<const float4 *>(u)[b * 8 + sub];
        v = make_float4(swiglu1(a.x, c.x), swiglu1(a.y, c.y), swiglu1(a.z, c.z), swiglu1(a.w, c.w));
    }
    float scale;
    int s;
    int packed = quantize4(v, &scale, &s);
    if (ok) {
        reinterpret_cast<int *>(qs)[b * 8 + sub] = packed;
        if (sub == 0) {
            scales[b] = scale;
            sums[b] = s;
        }
    }
}

// QActBatch::new of rms_norm(x) * w (tensor.rs:329-333, quant.rs:693-714),
// one workgroup per row of n floats (n % 32 == 0): the sum of squares over
// the thread's float4s in index order, then over the wave, then over the
// waves in order (as the GEMV's own staging of a normed input); h, when set,
// receives the normed row in f32.
__global__ __launch_bounds__(256) void norm_qact_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                       int n, float eps, float *__restrict__ h,
                                                       int8_t *__restrict__ qs, float *__restrict__ scales,
                                                       int32_t *__restrict__ sums) {
    __shared__ float s_ss[4];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & (WAVE - 1), wv = tid >> 6;
    const int n4 = n / 4, nb = n / BLOCK;
    const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)row * n);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    float ss = 0.0f;
    for (int i = tid; i < n4; i += 256) {
        const float4 v = xr[i];
        const float a = v.x * v.x, b = v.y * v.y, c = v.z * v.z, d = v.w * v.w;
        ss = ss + ((a + b) + (c + d));
    }
    ss = wave_sum(ss);
    if (lane == 0) s_ss[wv] = ss;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) t = t + s_ss[i];
    const float inv = 1.0f / sqrtf(t / (float)n + eps);
    // eight lanes per 32-block; every lane runs quantize4 (it swaps across lanes)
    for (int base = 0; base < n4; base += 256) {
        const int i = base + tid;
        const bool ok = i < n4;  // whole 8-lane groups: n4 % 8 == 0
        float4 v = ok ? xr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 g = ok ? w4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        v = make_float4((v.x * inv) * g.x, (v.y * inv) * g.y, (v.z * inv) * g.z, (v.w * inv) * g.w);
        float scale;
        int s;
        const int packed = quantize4(v, &scale, &s);
        if (ok) {
            if (h) reinterpret_cast<float4 *>(h + (size_t)row * n)[i] = v;
            reinterpret_cast<int *>(qs + (size_t)row * n)[i] = packed;
            if ((tid & 7) == 0) {
                scales[(size_t)row * nb + (i >> 3)] = scale;
                sums[(size_t)row * nb + (i >> 3)] = s;
            }
        }
    }
}


// One launch runs every job of the table.  Workgroups are spread over the
// jobs in proportion to their rows; each wave walks the row groups
// lw, lw + nw, ... of its job, loading the next group's weights before it
// computes the current one.  The first group's loads are issued before the
// activation is staged, so they fly while the workgroup quantises.  With
// The step's end (GreedyTail) in the head GEMV's last workgroup.  Each
// workgroup's choice and row 0's logit are stored at device scope (past the
// per-XCD L2) and have completed before the workgroup counts its arrival;
// the last to arrive reads them back at device scope -- no workgroup waits
// on another and no cache-wide fence is needed.  The best of the choices
// (the largest, the lowest index on ties) is the same in any reduction
// order.
template <int NWV>
__device__ void greedy_tail(const JobTable &tab, const GemvJob &job, int groups, float *s_av, int *s_ai) {
    __shared__ int s_last, s_best;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wv = tid >> 6;
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(tab.tail.arrivals, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (unsigned)groups - 1;
    __syncthreads();
    if (!s_last) return;
    float bv = -INFINITY;
    int bi = -1;
    for (int t = tid; t < groups; t += WAVE * NWV) {
        const float v = __hip_atomic_load(tab.arg_v + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int i = __hip_atomic_load(tab.arg_i + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi))) bv = v, bi = i;
    }
    for (int o = WAVE / 2; o > 0; o >>= 1) {
        const float v = __shfl_xor(bv, o);
        const int i = __shfl_xor(bi, o);
        if (i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi))) bv = v, bi = i;
    }
    if (lane == 0) s_av[wv] = bv, s_ai[wv] = bi;  // tid 0 read the entries before the last barrier
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < NWV; w++) {
            const float v = s_av[w];
            const int i = s_ai[w];
            if (i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi))) bv = v, bi = i;
        }
        const GreedyTail &e = tab.tail;
        // row 0 against the best of rows 1..: the first of equal maxima wins
        const float first = __hip_atomic_load(job.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int best = job.rows > 1 && first == first && bi >= 0 && bv > first ? bi : 0;
        s_best = best;
        *e.token = best;
        *e.pos = *e.pos + 1;
        const int k = *e.step;
        if (e.out && k < e.out_cap) e.out[k] = best;
        *e.step = k + 1;
        __hip_atomic_store(e.arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    const GreedyTail &e = tab.tail;
    const size_t r = (size_t)s_best;
    for (size_t k = tid; k < e.cols; k += WAVE * NWV) e.x[k] = dequant_elem(e.prec, e.qs, e.scales, e.cols, r, k);
}

// ROUTE, the router job (one workgroup, every router row) also keeps its
// outputs in LDS and its first wave routes them (MoE decode).
template <int PREC, int CPL, int R, int KIND, bool DOTS, bool WIDE = false, int NWV = WPB, bool ROUTE = false,
          bool PAIR = false>
__global__ __launch_bounds__(WAVE * NWV) void gemv_kernel(unsigned f0, unsigned f1, unsigned f2, unsigned f3,
                                                          const void *w_0, const float *ws_0, const float *xf_0,
                                                          const float *x2_0, int rows_0, unsigned colsnw_0,
                                                          JobTable tab) {
    static_assert(!PAIR || R % 2 == 0, "SwiGLU pairs take an even number of rows a step");
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ float s_lg[ROUTE ? MAX_EXPERTS : 1];  // the router's logits
    const int tid = threadIdx.x;
    const int lane = tid & (WAVE - 1);
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int blk = blockIdx.x;
    const int ji = job_of(tab, Firsts{{f0, f1, f2, f3}}, blk);
    const GemvJob &job = tab.j[ji];
    // What the first vector loads need: job 0's from the kernel's arguments
    // (preloaded into scalar registers, so a one-job launch issues its first
    // loads with no scalar load at all), other jobs' from the table in one
    // batch of scalar loads and one wait.  colsnw_0 = cols | nwaves << 16,
    // bit 30: every job stages job 0's input (the same activation and
    // columns), so any job's activation loads issue at once and its weight
    // fields' load overlaps them; bit 31: job 0 reads its weights through an
    // expert table, or is too large for the packing.
    const bool lead = !(colsnw_0 >> 31);
    const bool fast = ji == 0 && lead;
    const bool shared = lead && ((colsnw_0 >> 30) & 1u);
    const float *jxf, *jx2;
    int cols;
    if (fast || shared) {
        jxf = xf_0, jx2 = x2_0, cols = (int)(colsnw_0 & 0xffffu);
    } else {
        jxf = job.xf, jx2 = KIND == IN_SWIGLU ? job.xf2 : KIND == IN_NORM ? job.norm_w : nullptr, cols = job.cols;
        __asm__ volatile("" ::"s"(jxf), "s"(jx2), "s"(cols));
    }
    const int nb = cols / BLOCK;
    Stage<KIND, stage_batch(CPL, WIDE)> st;
    stage_load<KIND, stage_batch(CPL, WIDE), NWV>(job, jxf, jx2, st, nb, tid);
    __builtin_amdgcn_sched_barrier(0);  // the activation loads ahead of everything after
    const void *jw;
    const float *jws;
    int rows, nw, wave0;
    if (fast) {
        jw = w_0, jws = ws_0, rows = rows_0, nw = (int)((colsnw_0 >> 16) & 0x3fffu), wave0 = 0;
    } else {
        jw = job.w, jws = job.ws, rows = job.rows, nw = job.nwaves, wave0 = job.wave0;
        __asm__ volatile("" ::"s"(rows), "s"(nw), "s"(wave0), "s"(jw), "s"(jws), "s"(job.wtab));
    }
    const bool routes = ROUTE && ji == tab.route_job - 1;  // uniform per workgroup
    const bool argm = ji == tab.arg_job - 1;              // uniform per workgroup
    float arg_bv = -INFINITY;                             // the wave's greedy choice (lane 0)
    int arg_bi = -1;
    const int C = chunks_per_row(PREC, cols);
    const int nseg = (C + WAVE * CPL - 1) / (WAVE * CPL);
    const int PB = padded_blocks(PREC, C, CPL);
    const int ngroups = (rows + R - 1) / R;
    const int lw = (blk - wave0) * NWV + wv;  // this wave among the job's nw

    const int wrows = PAIR ? rows / 2 : rows;  // rows of each weight
    size_t wbytes = PREC == KH_Q8 ? (size_t)wrows * cols
                    : PREC == KH_Q4 ? (size_t)wrows * cols / 2
                                    : (size_t)wrows * (cols / QK_K) * Q4K_BYTES;
    const void *wp = jw;
    const float *wsp = jws;
    if (!fast && job.wtab) {  // an expert chosen on the device (MoE decode)
        // one address for the wave: the buffer descriptors stay in scalar registers
        const int x = __builtin_amdgcn_readfirstlane(*job.sel);
        wp = uniform_ptr(job.wtab[x]);
        wsp = uniform_ptr(job.wstab[x]);
    }
    const rsrc_t W = rsrc(wp, wbytes);
    const rsrc_t WS = rsrc(wsp, PREC == KH_Q4K ? 0 : (size_t)wrows * nb * 4);
    const rsrc_t W2 = PAIR ? rsrc(job.w2, wbytes) : W;
    const rsrc_t WS2 = PAIR ? rsrc(job.ws2, PREC == KH_Q4K ? 0 : (size_t)wrows * nb * 4) : WS;

    // the wave's work: its row groups, each cut into nseg segments, walked in
    // order; step s is group lw + (s / nseg) * nw, segment s % nseg.  Two
    // register buffers take even and odd steps: a step's loads are issued
    // just before the other buffer's step computes.  Every pass of the loop
    // issues the same loads (a step past the wave's work reads past the end
    // of the weights, which returns zeros), so each wait covers only the
    // loads it needs.  Step 0's loads fly while the workgroup stages the
    // activation.
    const int my_groups = lw < ngroups ? (ngroups - lw + nw - 1) / nw : 0;
    const int steps = my_groups * nseg;
    // loads are issued, and steps computed, in step order: each keeps a
    // cursor (its row group lw + k * nw and segment) instead of dividing
    int lk = 0, lseg = 0;
    auto load_step = [&](Chunks<PREC, CPL, R> &c) {
        __builtin_amdgcn_sched_barrier(0);
        load_chunks<PREC, CPL, R, PAIR>(c, W, WS, (lw + lk * nw) * R, cols, nb, lseg, lane, W2, WS2);
        __builtin_amdgcn_sched_barrier(0);
        if (++lseg == nseg) lseg = 0, lk++;
    };
    Chunks<PREC, CPL, R> ca, cb;
    load_step(ca);  // step 0
    // The bias and residual values of the wave's rows, lane k * R + i holding
    // those of row (lw + k * nw) * R + i: ahead of every later step's weights
    // (a load in the epilogue would wait for every weight load in flight),
    // behind step 0's, whose issue does not wait for these fields.
    const int my_rows = my_groups * R;
    const bool pre = my_rows <= WAVE;
    float pbias = 0.0f, pres = 0.0f;
    if (pre && (job.bias || job.accumulate)) {
        const int r = (lw + (lane / R) * nw) * R + lane % R;
        const unsigned off = lane < my_rows && r < rows ? (unsigned)r * 4u : 0xffffffffu;  // past the end: zero
        if (job.bias) pbias = bldf(rsrc(job.bias, (size_t)rows * 4), off);
        if (job.accumulate) pres = bldf(rsrc(job.y, (size_t)rows * 4), off);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- stage the activation in LDS (zero blocks pad the tail) ---------
    int8_t *sq = reinterpret_cast<int8_t *>(lds);
    float *ssc = reinterpret_cast<float *>(lds + (size_t)PB * 32);
    int *ssum = reinterpret_cast<int *>(ssc + PB);
    stage_activation<KIND, stage_batch(CPL, WIDE), NWV>(job, st, sq, ssc, ssum, PB, nb, cols, tid, lane, wv);
    __syncthreads();

    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++) acc[i] = 0.0f;
    // one step: the dot products of `c`, then (at a row group's last
    // segment) the rows' sums written out
    int k = 0, seg = 0;
    // The epilogue's fields, read once into scalar registers: read in the loop,
    // under the epilogue's conditions, each was a scalar load and a wait
    // every row group.
    float *const yo = job.y;
    const float *const bo = job.bias;
    const int accum = job.accumulate;
    const int y_atomic = routes && tab.route.arrivals ? 1 : 0;  // read back by another workgroup
    const int y0_atomic = argm && tab.tail.arrivals ? 1 : 0;     // row 0 likewise
    float *const y2o = PAIR ? job.y2 : nullptr;
    float *const ho = PAIR ? job.h : nullptr;
    __asm__ volatile("" ::"s"(yo), "s"(bo), "s"(accum), "s"(y_atomic), "s"(y0_atomic), "s"(y2o), "s"(ho));
    auto run_step = [&](const Chunks<PREC, CPL, R> &c) {
        const int r0 = (lw + k * nw) * R;
        compute_chunks<PREC, CPL, R, DOTS>(c, acc, sq, ssc, ssum, seg, lane, r0, rows, nb, C, job.dots);
        if (PAIR && seg == nseg - 1) {
            // gate row (r0 + i) / 2 and its up row: both, and swiglu of the pair
#pragma unroll
            for (int i = 0; i < R; i += 2) {
                const float g = wave_sum(acc[i]), u = wave_sum(acc[i + 1]);
                const int r = (r0 + i) >> 1;
                if (lane == 0 && r < wrows) {
                    yo[r] = g;
                    y2o[r] = u;
                    ho[r] = swiglu1(g, u);
                }
                acc[i] = 0.0f;
                acc[i + 1] = 0.0f;
            }
        } else if (seg == nseg - 1) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                const float v = wave_sum(acc[i]);
                const int r = r0 + i;
                float b = 0.0f, y0 = 0.0f;
                if (pre) {
                    b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pbias), k * R + i));
                    y0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pres), k * R + i));
                } else if (r < rows) {  // scalar loads: they wait on no weight load
                    if (bo) b = ((const_f32 *)bo)[r];
                    if (accum) y0 = ((const_f32 *)yo)[r];
                }
                if (lane == 0 && r < rows) {
                    float out = bo ? v + b : v;
                    if (accum) out = y0 + out;  // x += proj (llama.rs:273-276)
                    // read back by another workgroup: past the L2
                    if (y_atomic || (y0_atomic && r == 0))
                        __hip_atomic_store(yo + r, out, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    else
                        yo[r] = out;
                    if (routes) s_lg[r] = out;
                    // rows in increasing order: a later equal value never wins
                    if (argm && r >= 1 && out == out && (arg_bi < 0 || out > arg_bv)) arg_bv = out, arg_bi = r;
                }
                acc[i] = 0.0f;
            }
        }
        if (++seg == nseg) seg = 0, k++;
    };
    // Every way back to the top of the loop has issued the same loads in the
    // same order (the steps' loads in flight are always even, then odd), so
    // each step waits only for its own loads; the last steps leave the loop
    // by paths of their own and issue nothing past the wave's work.
    for (int step = 0; step < steps; step += 2) {
        load_step(cb);  // step + 1
        run_step(ca);   // step
        load_step(ca);  // step + 2
        if (step + 1 < steps) run_step(cb);
    }
    if (argm) {  // the workgroup's choice: its waves' in wave order, the lowest index on ties
        __shared__ float s_av[NWV];
        __shared__ int s_ai[NWV];
        if (lane == 0) s_av[wv] = arg_bv, s_ai[wv] = arg_bi;
        __syncthreads();
        if (tid == 0) {
            float bv = s_av[0];
            int bi = s_ai[0];
            for (int w = 1; w < NWV; w++) {
                const float v = s_av[w];
                const int i = s_ai[w];
                if (i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi))) bv = v, bi = i;
            }
            const int g = blk - wave0;
            if (tab.tail.arrivals) {  // read back by the last workgroup: past the L2
                __hip_atomic_store(tab.arg_v + g, bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(tab.arg_i + g, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                tab.arg_v[g] = bv;
                tab.arg_i[g] = bi;
            }
            if (g == 0) *tab.arg_n = nw / NWV;
        }
        if (tab.tail.arrivals) greedy_tail<NWV>(tab, job, nw / NWV, s_av, s_ai);
    }
    if constexpr (ROUTE) {
        if (routes && tab.route.arrivals) {
            // The router's rows are spread over route.groups workgroups; the
            // last to finish routes.  Each wave's logit stores (device scope,
            // past the per-XCD L2) have completed before the workgroup counts
            // its arrival, and the last reads them back at device scope, so no
            // cache-wide fence is needed.  Nothing waits on another
            // workgroup: every workgroup counts itself once and leaves.
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (wv == 0) {
                unsigned old = 0;
                if (lane == 0)
                    old = __hip_atomic_fetch_add(tab.route.arrivals, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                old = (unsigned)__builtin_amdgcn_readfirstlane((int)old);
                if (old == (unsigned)tab.route.groups - 1) {
                    for (int i = lane; i < rows; i += WAVE)
                        s_lg[i] = __hip_atomic_load(job.y + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    wave_lds_sync();
                    route_one(tab.route, 0, s_lg);
                    if (lane == 0) __hip_atomic_store(tab.route.arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        } else if (routes) {
            __syncthreads();  // every wave's logits are in LDS
            if (wv == 0) route_one(tab.route, 0, s_lg);
        }
    }
}

// f32 weights: tensor::matvec_bt (tensor.rs:56-79); lanes stride the row
// four weights at a time, x read through the cache.
__global__ __launch_bounds__(256) void gemv_f32_kernel(JobTable tab) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int blk = blockIdx.x;
    const GemvJob &job = tab.j[job_of(tab, blk)];
    const int rows = job.rows, cols = job.cols;
    const int lw = (blk - job.wave0) * WAVES_PER_BLOCK + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const float *W = static_cast<const float *>(job.w);
    for (int r = lw; r < rows; r += job.nwaves) {
        const float *wr = W + (size_t)r * cols;
        float s = 0.0f;
        if ((cols & 3) == 0) {
            for (int g = lane; g < cols / 4; g += WAVE) {
                float4 a = reinterpret_cast<const float4 *>(wr)[g];
                float4 b = reinterpret_cast<const float4 *>(job.xf)[g];
                s = fmaf(a.x, b.x, s);
                s = fmaf(a.y, b.y, s);
                s = fmaf(a.z, b.z, s);
                s = fmaf(a.w, b.w, s);
            }
        } else {
            for (int k = lane; k < cols; k += WAVE) s = fmaf(wr[k], job.xf[k], s);
        }
        const float v = wave_sum(s);
        if (lane == 0) {
            float out = job.bias ? v + job.bias[r] : v;
            if (job.accumulate) out = job.y[r] + out;
            job.y[r] = out;
        }
    }
}

// ---------------------------------------------------------------------------
// Several tokens at once: matmul_bt for m <= MULTI_MAX rows (batched decode,
// quant.rs:751-907).  The weights stream from HBM once for all m tokens; each
// chunk's weight codes and scales are decoded once and dotted with every
// token's codes, staged side by side in LDS.  Per token the arithmetic is the
// single-token kernel's, term for term, so token t's row equals a GEMV of
// that token to the bit.
// ---------------------------------------------------------------------------


// Weights that read the same rows of codes (q/k/v, gate/up) in one launch:
// the workgroups are dealt to the jobs in proportion to their rows.
struct MultiJob {
    const void *w;
    const float *ws;
    const float *bias;    // [rows] or null
    float *y;             // [m][rows]
    int rows;
    int accumulate;       // y += x W^T (+ bias): the residual add
    int wg0, nwaves;      // set by the launcher: the job's first workgroup, its waves
};

struct MultiArgs {
    const int8_t *xq;     // [m][cols] codes
    const float *xs;      // [m][cols / 32]
    const int32_t *xsum;  // [m][cols / 32]
    const float *xf;      // or, when set: [m][cols] f32 rows each workgroup quantises itself
    int cols, m, njobs;
    MultiJob j[MULTI_JOBS];
};

// The chunks' contribution to each token's accumulator (one row per step).
template <int PREC, int CPL, int T>
__device__ __forceinline__ void compute_multi(const Chunks<PREC, CPL, 1> &c, float (&acc)[T], const int8_t *sq,
                                              const float *ssc, const int *ssum, int PB, int seg, int lane) {
    const int gl = seg * WAVE * CPL + lane;
    if constexpr (PREC == KH_Q8) {
#pragma unroll
        for (int t = 0; t < CPL; t++) {
            const int g = gl + t * WAVE;
            const int4 w = c.w[0][t];
#pragma unroll
            for (int k = 0; k < T; k++) {
                const int4 a = *reinterpret_cast<const int4 *>(sq + (size_t)k * PB * 32 + g * 16);
                const float as = ssc[k * PB + (g >> 1)];
                int d = dot4(w.x, a.x, 0);
                d = dot4(w.y, a.y, d);
                d = dot4(w.z, a.z, d);
                d = dot4(w.w, a.w, d);
                d += dpp<DPP_XOR1>(d);
                float sc = c.s[0][t] * as;
                sc = sc * (float)d;
                acc[k] += (lane & 1) ? 0.0f : sc;
            }
        }
    } else if constexpr (PREC == KH_Q4) {
#pragma unroll
        for (int t = 0; t < CPL; t++) {
            const int g = gl + t * WAVE;
            const int4 q = c.w[0][t];
            const int4 lo4 = {q.x & 0x0f0f0f0f, q.y & 0x0f0f0f0f, q.z & 0x0f0f0f0f, q.w & 0x0f0f0f0f};
            const int4 hi4 = {(q.x >> 4) & 0x0f0f0f0f, (q.y >> 4) & 0x0f0f0f0f, (q.z >> 4) & 0x0f0f0f0f,
                              (q.w >> 4) & 0x0f0f0f0f};
#pragma unroll
            for (int k = 0; k < T; k++) {
                const int8_t *sk = sq + (size_t)k * PB * 32;
                const int4 alo = *reinterpret_cast<const int4 *>(sk + g * 32);
                const int4 ahi = *reinterpret_cast<const int4 *>(sk + g * 32 + 16);
                const float as = ssc[k * PB + g];
                const int asum = ssum[k * PB + g];
                int lo = dot4(lo4.x, alo.x, 0);
                lo = dot4(lo4.y, alo.y, lo);
                lo = dot4(lo4.z, alo.z, lo);
                lo = dot4(lo4.w, alo.w, lo);
                int hi = dot4(hi4.x, ahi.x, 0);
                hi = dot4(hi4.y, ahi.y, hi);
                hi = dot4(hi4.z, ahi.z, hi);
                hi = dot4(hi4.w, ahi.w, hi);
                const int d = lo + hi - 8 * asum;  // quant.rs:187
                float sc = c.s[0][t] * as;
                sc = sc * (float)d;
                acc[k] += sc;
            }
        }
    } else {
        const int half = lane & 1, cc = (lane & 7) >> 1, j = 2 * cc + half;
        const Q4kLane L = q4k_lane(j);
#pragma unroll
        for (int t = 0; t < CPL; t++) {
            const int g = gl + t * WAVE;
            const int b0 = (g >> 3) * 8 + 2 * cc;
            const int4 q = c.w[0][t];
            const int4 lo4 = {q.x & 0x0f0f0f0f, q.y & 0x0f0f0f0f, q.z & 0x0f0f0f0f, q.w & 0x0f0f0f0f};
            const int4 hi4 = {(q.x >> 4) & 0x0f0f0f0f, (q.y >> 4) & 0x0f0f0f0f, (q.z >> 4) & 0x0f0f0f0f,
                              (q.w >> 4) & 0x0f0f0f0f};
            const int4 h = c.h[0][t];
            unsigned scb, mnb;
            q4k_scale_min_bfe(h, L, scb, mnb);
            const float dl = half_bits_to_float((unsigned)h.x) * (float)scb;
            const float ml = half_bits_to_float((unsigned)h.x >> 16) * (float)mnb;
#pragma unroll
            for (int k = 0; k < T; k++) {
                const int8_t *sk = sq + (size_t)k * PB * 32;
                const int4 alo = *reinterpret_cast<const int4 *>(sk + b0 * 32 + 16 * half);
                const int4 ahi = *reinterpret_cast<const int4 *>(sk + (b0 + 1) * 32 + 16 * half);
                const float as = ssc[k * PB + b0 + half];
                const int asum = ssum[k * PB + b0 + half];
                int lo = dot4(lo4.x, alo.x, 0);
                lo = dot4(lo4.y, alo.y, lo);
                lo = dot4(lo4.z, alo.z, lo);
                lo = dot4(lo4.w, alo.w, lo);
                int hi = dot4(hi4.x, ahi.x, 0);
                hi = dot4(hi4.y, ahi.y, hi);
                hi = dot4(hi4.z, ahi.z, hi);
                hi = dot4(hi4.w, ahi.w, hi);
                lo += dpp<DPP_XOR1>(lo);
                hi += dpp<DPP_XOR1>(hi);
                const int d = half ? hi : lo;
                // the single-token kernel's roundings (compute_chunks): ml * asum,
                // dl * d less that, then into the row, each rounded once
                const float t2 = __builtin_fmaf(ml, (float)asum, -0.0f);
                const float sc = __builtin_fmaf(dl, (float)d, -t2);
                acc[k] = __builtin_fmaf(as, sc, acc[k]);
            }
        }
    }
}

// One wave per row at a time, rows lw, lw + nw, ...; each row in nseg
// segments of CPL chunks per lane.  T >= m token slots (unused ones meet
// zero codes).  The workgroup stages every token's codes first (the weights
// of its first step are requested right after, so they fly while the
// workgroup waits on the stage).
template <int PREC, int CPL, int T>
__global__ __launch_bounds__(WAVE * WPB) void gemv_multi_kernel(unsigned g12, MultiArgs a) {
    static_assert(MULTI_JOBS == 3, "g12 holds jobs 1 and 2");
    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = threadIdx.x, lane = tid & (WAVE - 1);
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ji = ((int)blockIdx.x >= (int)(g12 & 0xffffu) ? 1 : 0) + ((int)blockIdx.x >= (int)(g12 >> 16) ? 1 : 0);
    const MultiJob &job = a.j[ji];
    // the fields the first loads need, in one batch of scalar loads
    __asm__ volatile("" ::"s"(job.w), "s"(job.ws), "s"(job.rows), "s"(job.wg0), "s"(job.nwaves), "s"(a.cols),
                     "s"(a.m), "s"(a.xq), "s"(a.xs), "s"(a.xsum), "s"(a.xf));
    const int rows = job.rows, cols = a.cols, nb = cols / BLOCK;
    const int C = chunks_per_row(PREC, cols);
    const int nseg = (C + WAVE * CPL - 1) / (WAVE * CPL);
    const int PB = padded_blocks(PREC, C, CPL);
    const int nw = job.nwaves, lw = ((int)blockIdx.x - job.wg0) * WPB + wv;
    const int my_rows = lw < rows ? (rows - lw + nw - 1) / nw : 0;
    const int steps = my_rows * nseg;

    int8_t *sq = reinterpret_cast<int8_t *>(lds);
    float *ssc = reinterpret_cast<float *>(lds + (size_t)T * PB * 32);
    int *ssum = reinterpret_cast<int *>(ssc + (size_t)T * PB);
    if (a.xf) {
        // f32 rows quantised here as QActBatch::new does (quant.rs:682-738),
        // 8 lanes per 32-block as qact_kernel: the same codes, scales and
        // sums.  float4 i: token i / (8 PB), float4 i % (8 PB) of its padded
        // row; a group of 8 lanes is always whole (the stride is a multiple
        // of 8), and padding quantises to zeros.
        const rsrc_t X = rsrc(a.xf, (size_t)a.m * cols * 4);
        for (int i = tid; i < T * PB * 8; i += WAVE * WPB) {
            const int k = i / (PB * 8), c = i % (PB * 8);
            const bool ok = k < a.m && c < nb * 8;
            const float4 v = __builtin_bit_cast(float4, bld16(X, ok ? (unsigned)((k * cols + c * 4) * 4) : 0xffffffffu));
            float scale;
            int sum;
            reinterpret_cast<int *>(sq)[i] = quantize4(v, &scale, &sum);
            if ((tid & 7) == 0) {
                ssc[i >> 3] = scale;
                ssum[i >> 3] = sum;
            }
        }
    } else {
        const rsrc_t Q = rsrc(a.xq, (size_t)a.m * cols), S = rsrc(a.xs, (size_t)a.m * nb * 4),
                     M = rsrc(a.xsum, (size_t)a.m * nb * 4);
        for (int i = tid; i < T * PB * 2; i += WAVE * WPB) {  // int4 i: token i / (2 PB), 16 bytes
            const int k = i / (PB * 2), c = i % (PB * 2);
            const bool ok = k < a.m && c < nb * 2;
            const int4 v = bld16(Q, ok ? (unsigned)(k * cols + c * 16) : 0xffffffffu);
            reinterpret_cast<int4 *>(sq)[i] = v;
        }
        for (int i = tid; i < T * PB; i += WAVE * WPB) {
            const int k = i / PB, b = i % PB;
            const bool ok = k < a.m && b < nb;
            const unsigned off = ok ? (unsigned)((k * nb + b) * 4) : 0xffffffffu;
            ssc[i] = bldf(S, off);
            ssum[i] = bldi(M, off);
        }
    }

    const size_t wbytes = PREC == KH_Q8 ? (size_t)rows * cols
                          : PREC == KH_Q4 ? (size_t)rows * cols / 2
                                          : (size_t)rows * (cols / QK_K) * Q4K_BYTES;
    const rsrc_t W = rsrc(job.w, wbytes);
    const rsrc_t WS = rsrc(job.ws, PREC == KH_Q4K ? 0 : (size_t)rows * nb * 4);
    auto load_step = [&](Chunks<PREC, CPL, 1> &c, int s) {
        __builtin_amdgcn_sched_barrier(0);
        load_chunks<PREC, CPL, 1>(c, W, WS, lw + (s / nseg) * nw, cols, nb, s % nseg, lane, W, WS);
        __builtin_amdgcn_sched_barrier(0);
    };
    Chunks<PREC, CPL, 1> ca, cb;
    load_step(ca, 0);
    __syncthreads();

    float acc[T];
#pragma unroll
    for (int k = 0; k < T; k++) acc[k] = 0.0f;
    auto run_step = [&](const Chunks<PREC, CPL, 1> &c, int step) {
        const int r = lw + (step / nseg) * nw, seg = step % nseg;
        compute_multi<PREC, CPL, T>(c, acc, sq, ssc, ssum, PB, seg, lane);
        if (seg == nseg - 1) {
            const float b = job.bias && r < rows ? ((const_f32 *)job.bias)[r] : 0.0f;
#pragma unroll
            for (int k = 0; k < T; k++) {
                const float v = wave_sum(acc[k]);
                if (lane == 0 && r < rows && k < a.m) {
                    float *dst = job.y + (size_t)k * rows + r;
                    const float o = job.bias ? v + b : v;
                    *dst = job.accumulate ? *dst + o : o;  // x += proj (llama.rs:273-276)
                }
                acc[k] = 0.0f;
            }
        }
    };
    // the single-token kernel's loop: the same loads on every pass
    for (int step = 0; step < steps; step += 2) {
        load_step(cb, step + 1);
        run_step(ca, step);
        load_step(ca, step + 2);
        if (step + 1 < steps) run_step(cb, step + 1);
    }
}

struct Plan {
    int cpl, r, wg;  // chunks per lane per segment, rows per wave-step, workgroups per CU
    int nwv;         // waves per workgroup
};

// Launch shape from sweeps over Llama-3-8B and Qwen2.5-0.5B shapes with
// weights far larger than the cache.  Q4_K: short steps pipeline best -- one
// chunk per lane (two segments per 4096-wide row) and two rows per step, or
// two chunks per lane and one row for wide rows, three workgroups per CU (one
// for wide activations, which every workgroup stages).  q8/q4: a row per
// segment, R = 4 rows per step for rows of one chunk a lane, 2 for four,
// 1 for two, three or five and more (and for very tall launches, where
// balance across waves matters more), fewer for short matrices so there are
// enough waves, two workgroups per CU (three when very tall).
Plan plan_for(int prec, int maxC, int maxCols, int rows_total, int cu_count) {
    int cpl = (maxC + WAVE - 1) / WAVE;
    if (cpl < 1) cpl = 1;
    if (cpl > 8) cpl = 8;  // wider rows take several segments
    int r, wg, nwv = WPB;
    if (prec == KH_Q4K) {
        cpl = cpl <= 2 ? 1 : 2;
        r = cpl == 1 ? 2 : 1;
        wg = maxCols >= 8192 ? 1 : 3;
    } else {
        const bool tall = rows_total >= 16384 && cpl >= 2;
        // rows of two or three chunks a lane (1025-3072 columns:
        // DeepSeek-V2-Lite's MoE layer, 1408 / 2048 / 2816) one row a step:
        // 44.3 -> 42.9 us per decode layer
        r = cpl == 1 ? 4 : cpl <= 3 ? 1 : cpl == 4 ? 2 : 1;
        if (tall) r = 1;
        wg = tall ? 3 : 2;
    }
    // short matrices: fewer rows per wave, more waves
    while (r > 1 && (rows_total + r - 1) / r < nwv * cu_count) r /= 2;
    // tuning knobs
    const int fc = env_int("KVAD_GEMV_CPL", 0);  // chunks per lane (more segments when fewer)
    if (fc > 0 && fc <= 8) cpl = fc;
    const int forced = env_int("KVAD_GEMV_R", 0);
    if (forced == 1 || (forced == 2 && cpl <= 4) || (forced == 4 && cpl <= 2)) r = forced;
    const int fw = env_int("KVAD_GEMV_WG_PER_CU", 0);
    if (fw > 0) wg = fw;
    // A wide Q4_K activation, staged by every workgroup: one workgroup of 16
    // waves per CU stages it once, with twice the threads (one staging
    // batch of four loads per thread covers up to 16384 columns).
    if (prec == KH_Q4K && cpl == 2 && r == 1 && maxCols >= 8192 && maxCols <= 16384) nwv = 16;
    if (env_int("KVAD_GEMV_WAVES", 0) == 8) nwv = WPB;
    return {cpl, r, wg, nwv};
}

template <int PREC, int CPL, int R, int KIND, bool WIDE, int NWV>
void launch_one(kh_ctx *ctx, const JobTable &tab, int blocks, size_t lds) {
    const Firsts fp = packed_first(tab);
    const Lead ld = lead_job(tab);
    hipLaunchKernelGGL((gemv_kernel<PREC, CPL, R, KIND, false, WIDE, NWV>), dim3(blocks), dim3(WAVE * NWV), lds,
                       ctx->stream, fp.f[0], fp.f[1], fp.f[2], fp.f[3], ld.w, ld.ws, ld.xf, ld.x2, ld.rows, ld.colsnw, tab);
}

template <int PREC, int CPL, int R, bool WIDE, int NWV = WPB>
void launch_kind(kh_ctx *ctx, const JobTable &tab, int blocks, size_t lds, int kind) {
    if (kind == IN_F32) launch_one<PREC, CPL, R, IN_F32, WIDE, NWV>(ctx, tab, blocks, lds);
    else if (kind == IN_SWIGLU) launch_one<PREC, CPL, R, IN_SWIGLU, WIDE, NWV>(ctx, tab, blocks, lds);
    else if (kind == IN_NORM) launch_one<PREC, CPL, R, IN_NORM, WIDE, NWV>(ctx, tab, blocks, lds);
    else launch_one<PREC, CPL, R, IN_CODES, WIDE, NWV>(ctx, tab, blocks, lds);
}

template <int PREC, int CPL, int R>
void launch_pair(kh_ctx *ctx, const JobTable &tab, int blocks, size_t lds, int kind) {
    const Firsts fp = packed_first(tab);
    const Lead ld = lead_job(tab);
    if (kind == IN_NORM)
        hipLaunchKernelGGL((gemv_kernel<PREC, CPL, R, IN_NORM, false, false, WPB, false, true>), dim3(blocks),
                           dim3(WAVE * WPB), lds, ctx->stream, fp.f[0], fp.f[1], fp.f[2], fp.f[3], ld.w, ld.ws, ld.xf, ld.x2, ld.rows, ld.colsnw, tab);
    else
        hipLaunchKernelGGL((gemv_kernel<PREC, CPL, R, IN_F32, false, false, WPB, false, true>), dim3(blocks),
                           dim3(WAVE * WPB), lds, ctx->stream, fp.f[0], fp.f[1], fp.f[2], fp.f[3], ld.w, ld.ws, ld.xf, ld.x2, ld.rows, ld.colsnw, tab);
}

template <int PREC>
int launch_prec(kh_ctx *ctx, JobTable &tab, int maxC, int maxCols, int rows_total, bool dots, int kind) {
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    Plan p = plan_for(PREC, maxC, maxCols, rows_total, cu);
    if (dots) p = {8, 1, 2, WPB};  // block dots (a debugging aid): one kernel shape serves every width
    // a SwiGLU pair takes its rows two at a time: an even number a step
    const bool pair = tab.j[0].w2 != nullptr;
    if (pair) {
        if (tab.n != 1 || dots || tab.route_job || tab.arg_job || tab.j[0].bias || tab.j[0].accumulate ||
            tab.j[0].rows % 2 || (kind != IN_NORM && kind != IN_F32))
            return fail(KH_EINVAL, "matvec: a SwiGLU pair is its launch's only job, without bias or residual");
        if (p.cpl > 4) return fail(KH_DECLINED, "matvec: no SwiGLU-pair kernel for rows this wide");
        // one gate/up pair a step: Qwen2.5-0.5B's 2 x 4864 q8 rows of 896
        // columns take 6.7 us this way against 7.9 us at two pairs a step
        p.r = env_int("KVAD_GEMV_R", 0) == 4 && p.cpl <= 2 ? 4 : 2;
        p.nwv = WPB;
    }
    for (int i = 0; i < tab.n; i++) {
        size_t wb = (size_t)tab.j[i].rows * tab.j[i].cols;
        if (wb >= 0xfff00000ull) return fail(KH_DECLINED, "matvec: weights of 4 GiB or more are not addressed here");
    }
    // workgroups: about `wg_per_cu` per CU over the launch, shared out by rows
    const int cap_wg = p.wg * cu;
    int blocks = 0;
    for (int i = 0; i < tab.n; i++) {
        const int groups = (tab.j[i].rows + p.r - 1) / p.r;
        const int want = (groups + p.nwv - 1) / p.nwv;
        int share = (int)((long long)cap_wg * tab.j[i].rows / (rows_total > 0 ? rows_total : 1));
        if (share < 1) share = 1;
        // the router: one workgroup, or (counting arrivals) as many as its rows need
        int nwg = want < share ? want : share;
        if (i == tab.route_job - 1) {
            nwg = tab.route.arrivals ? want : 1;
            tab.route.groups = nwg;
        }
        tab.j[i].wave0 = blocks;  // first workgroup of the job
        tab.j[i].nwaves = nwg * p.nwv;
        blocks += nwg;
    }
    set_first(tab);
    if (blocks == 0) return KH_OK;
    if (blocks >= 0xffff) return fail(KH_DECLINED, "matvec: 65535 workgroups or more in one launch");
    if (tab.arg_job && tab.j[tab.arg_job - 1].nwaves / p.nwv > tab.arg_cap)
        return fail(KH_DECLINED, "matvec: more workgroups than greedy partials");
    const int pb = padded_blocks(PREC, maxC, p.cpl);
    const size_t lds = (size_t)pb * 32 + 8 * (size_t)pb;
    if (lds > 64 * 1024) return fail(KH_DECLINED, "matvec: activation too wide for the LDS stage");
    // rows of several segments with R == 1 and CPL < 4 have a WIDE build
    const bool wide = !stage_fits(kind, pb, stage_batch(p.cpl, false), p.nwv);
    if (wide && !(p.cpl >= 4 || (p.r == 1 && stage_fits(kind, pb, stage_batch(p.cpl, true), p.nwv))))
        return fail(KH_DECLINED, "matvec: an f32 activation this wide is quantised in a launch of its own");
    if (pair) {
        if (wide) return fail(KH_DECLINED, "matvec: no SwiGLU-pair kernel for an input this wide");
#define KH_PAIR(CPL, R)                                                       \
    if (p.cpl == CPL && p.r == R) {                                           \
        launch_pair<PREC, CPL, R>(ctx, tab, blocks, lds, kind);               \
        KH_HIP(hipGetLastError());                                            \
        return KH_OK;                                                         \
    }
        KH_PAIR(1, 4) KH_PAIR(1, 2) KH_PAIR(2, 4) KH_PAIR(2, 2) KH_PAIR(3, 2) KH_PAIR(4, 2)
#undef KH_PAIR
        return fail(KH_DECLINED, "matvec: no SwiGLU-pair kernel for this plan");
    }
    if (dots) {
        dim3 grid(blocks), block(WAVE * WPB);
        const Firsts fp = packed_first(tab);
    const Lead ld = lead_job(tab);
        if (kind == IN_CODES)
            hipLaunchKernelGGL((gemv_kernel<PREC, 8, 1, IN_CODES, true>), grid, block, lds, ctx->stream, fp.f[0],
                               fp.f[1], fp.f[2], fp.f[3], ld.w, ld.ws, ld.xf, ld.x2, ld.rows, ld.colsnw, tab);
        else if (kind == IN_F32)
            hipLaunchKernelGGL((gemv_kernel<PREC, 8, 1, IN_F32, true>), grid, block, lds, ctx->stream, fp.f[0],
                               fp.f[1], fp.f[2], fp.f[3], ld.w, ld.ws, ld.xf, ld.x2, ld.rows, ld.colsnw, tab);
        else
            return fail(KH_EINVAL, "matvec: block dots are offered for plain and pre-quantised inputs only");
        KH_HIP(hipGetLastError());
        return KH_OK;
    }
#define KH_CASE(CPL, R)                                                       \
    if (p.cpl == CPL && p.r == R && !wide) {                                  \
        launch_kind<PREC, CPL, R, false>(ctx, tab, blocks, lds, kind);        \
        KH_HIP(hipGetLastError());                                            \
        return KH_OK;                                                         \
    }
#define KH_WIDE(CPL)                                                          \
    if (p.cpl == CPL && p.r == 1 && wide) {                                   \
        launch_kind<PREC, CPL, 1, true>(ctx, tab, blocks, lds, kind);         \
        KH_HIP(hipGetLastError());                                            \
        return KH_OK;                                                         \
    }
    if (tab.route_job) {  // the MoE decode step's router with its routing
        const Firsts fpr = packed_first(tab);
        const Lead ld = lead_job(tab);
#define KH_ROUTE(CPL, R)                                                                                       \
    if (p.cpl == CPL && p.r == R) {                                                                            \
        hipLaunchKernelGGL((gemv_kernel<PREC, CPL, R, IN_F32, false, false, WPB, true>), dim3(blocks),         \
                           dim3(WAVE * WPB), lds, ctx->stream, fpr.f[0], fpr.f[1], fpr.f[2], fpr.f[3], ld.w, ld.ws, ld.xf, ld.x2, ld.rows, ld.colsnw, tab);   \
        KH_HIP(hipGetLastError());                                                                             \
        return KH_OK;                                                                                          \
    }
        if constexpr (PREC == KH_Q8) {
            if (kind == IN_F32 && !wide && p.nwv == WPB) {
                KH_ROUTE(1, 4) KH_ROUTE(1, 2) KH_ROUTE(2, 2) KH_ROUTE(2, 1) KH_ROUTE(4, 1)
            }
        }
#undef KH_ROUTE
        return fail(KH_DECLINED, "matvec: no routing kernel for this plan");
    }
    if (p.nwv == 16) {
        if (p.cpl != 2 || p.r != 1 || wide) return fail(KH_EINVAL, "matvec: no 16-wave kernel for this plan");
        launch_kind<PREC, 2, 1, false, 16>(ctx, tab, blocks, lds, kind);
        KH_HIP(hipGetLastError());
        return KH_OK;
    }
    KH_CASE(1, 4) KH_CASE(1, 2) KH_CASE(1, 1)
    KH_CASE(2, 4) KH_CASE(2, 2) KH_CASE(2, 1)
    KH_CASE(3, 2) KH_CASE(3, 1) KH_CASE(4, 2) KH_CASE(4, 1)
    KH_CASE(5, 1) KH_CASE(6, 1) KH_CASE(7, 1) KH_CASE(8, 1)
    KH_WIDE(1) KH_WIDE(2) KH_WIDE(3)
#undef KH_CASE
#undef KH_WIDE
    return fail(KH_EINVAL, "matvec: no kernel for this plan");
}

int launch_f32(kh_ctx *ctx, JobTable &tab) {
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    int blocks = 0;
    for (int i = 0; i < tab.n; i++) {
        int nw = tab.j[i].rows < 8 * cu ? tab.j[i].rows : 8 * cu;
        tab.j[i].wave0 = blocks;
        tab.j[i].nwaves = nw;
        blocks += (nw + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
    }
    set_first(tab);
    if (blocks == 0) return KH_OK;
    hipLaunchKernelGGL(gemv_f32_kernel, dim3(blocks), dim3(256), 0, ctx->stream, tab);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

// ---------------------------------------------------------------------------
// small kernels
// ---------------------------------------------------------------------------

__global__ void fill_kernel(float *p, size_t n, float value) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = value;
}

// Weight::row (quant.rs:374-402) and the Q4_K decoder (mpp.rs:304-315).
// ---- the streaming ceiling of a launch (a timing aid) ----------------------
// The bytes of up to STREAM_ARRAYS device arrays read once with 16-byte
// loads and no arithmetic: workgroup b takes the L * blockDim consecutive
// 16-byte units from b * L * blockDim, each lane issuing all L of its loads
// (consecutive lanes on consecutive units) before it waits; each lane folds
// what it read into one word and each workgroup writes one word of `sink`.
// No activation and no arithmetic: the same launch structure as the GEMV it
// is set beside, with every byte in flight as early as it can be.
constexpr int STREAM_ARRAYS = 8;
struct StreamArgs {
    const void *p[STREAM_ARRAYS];
    unsigned end[STREAM_ARRAYS];  // prefix sums of the arrays' 16-byte units
    int n;
    unsigned total;
    unsigned *sink;
};

// The first three arrays, their ends, the count, the total and the sink come
// as the kernel's first arguments, preloaded into scalar registers as the
// GEMV's first job is, so the probe pays no more scalar loads than the GEMV
// before its first load; arrays 3.. are read from `a`.
template <int L, int AUX>
__global__ __launch_bounds__(1024) void stream_kernel(const void *p0, const void *p1, const void *p2, unsigned e0,
                                                      unsigned e1, unsigned e2, int n, unsigned total,
                                                      unsigned *sink, StreamArgs a) {
    const unsigned T = blockDim.x, base = blockIdx.x * T * L + threadIdx.x;
    int4 v[L];
#pragma unroll
    for (int u = 0; u < L; u++) {
        const unsigned i = base + (unsigned)u * T;
        int k = (n > 1 && i >= e0 ? 1 : 0) + (n > 2 && i >= e1 ? 1 : 0);
        const void *p = k == 0 ? p0 : k == 1 ? p1 : p2;
        unsigned lo = k == 0 ? 0u : k == 1 ? e0 : e1, hi = k == 0 ? e0 : k == 1 ? e1 : e2;
        if (n > 3 && i >= e2) {  // array 3 or later
            k = 3;
#pragma unroll
            for (int j = 3; j < STREAM_ARRAYS - 1; j++) k += (j < n - 1 && i >= a.end[j]) ? 1 : 0;
            p = a.p[k];
            lo = a.end[k - 1];
            hi = a.end[k];
        }
        const rsrc_t r = rsrc(p, (size_t)(hi - lo) * 16);
        v[u] = i < total ? __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(r, (i - lo) * 16u, 0, AUX))
                         : make_int4(0, 0, 0, 0);
    }
    unsigned fold = 0;
#pragma unroll
    for (int u = 0; u < L; u++) fold ^= (unsigned)(v[u].x ^ v[u].y ^ v[u].z ^ v[u].w);
    fold = wave_xor(fold);
    __shared__ unsigned s_f[16];
    if ((threadIdx.x & (WAVE - 1)) == 0) s_f[threadIdx.x >> 6] = fold;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned f = 0;
        for (int w = 0; w < (int)(blockDim.x >> 6); w++) f ^= s_f[w];
        sink[blockIdx.x & (STREAM_SINK - 1)] = f;
    }
}

// Row r_dev[y] (or r_host) of the weight into out row y, one grid row each.
__global__ void dequant_row_kernel(int prec, const void *qs, const float *scales, size_t cols, size_t r_host,
                                   const int32_t *r_dev,
                                   float *out) {
    const size_t r = r_dev ? (size_t)r_dev[blockIdx.y] : r_host;
    size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= cols) return;
    out[(size_t)blockIdx.y * cols + k] = dequant_elem(prec, qs, scales, cols, r, k);
}

}  // namespace

int launch_qact(kh_ctx *ctx, const float *x, size_t m, size_t k, const QAct &out) {
    size_t nblocks = m * k / BLOCK;
    if (nblocks == 0) return KH_OK;
    size_t threads = nblocks * 8;
    dim3 grid((unsigned)((threads + 255) / 256)), block(256);
    hipLaunchKernelGGL(qact_kernel, grid, block, 0, ctx->stream, x, nblocks, out.qs, out.scales, out.sums);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int launch_quant_check(kh_ctx *ctx, unsigned long long *counts) {
    hipLaunchKernelGGL(quant_check_kernel, dim3(8192), dim3(256), 0, ctx->stream, counts);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int launch_norm_qact(kh_ctx *ctx, const float *x, const float *w, size_t m, size_t n, float eps, float *h,
                     const QAct &out) {
    if (m == 0 || n == 0) return KH_OK;
    if (n % BLOCK || n > 0x7fffffff || m > 0x7fffffff) return fail(KH_EINVAL, "norm_qact: n must be a multiple of 32");
    hipLaunchKernelGGL(norm_qact_kernel, dim3((unsigned)m), dim3(256), 0, ctx->stream, x, w, (int)n, eps, h, out.qs,
                       out.scales, out.sums);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int launch_swiglu_qact(kh_ctx *ctx, const float *g, const float *u, size_t m, size_t k, const QAct &out) {
    size_t nblocks = m * k / BLOCK;
    if (nblocks == 0) return KH_OK;
    size_t threads = nblocks * 8;
    hipLaunchKernelGGL(swiglu_qact_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, ctx->stream, g, u,
                       nblocks, out.qs, out.scales, out.sums);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

template <int PREC, int T>
int launch_multi_t(kh_ctx *ctx, const MultiArgs &a, int cpl, int blocks, size_t lds) {
    if (blocks >= 0xffff) return fail(KH_DECLINED, "matmul: 65535 workgroups or more in one launch");
    dim3 grid(blocks), block(WAVE * WPB);
    if (cpl == 1)
        hipLaunchKernelGGL((gemv_multi_kernel<PREC, 1, T>), grid, block, lds, ctx->stream,
                           multi_firsts(a.njobs, a.j[1].wg0, a.j[2].wg0), a);
    else
        hipLaunchKernelGGL((gemv_multi_kernel<PREC, 2, T>), grid, block, lds, ctx->stream,
                           multi_firsts(a.njobs, a.j[1].wg0, a.j[2].wg0), a);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

template <int PREC>
int launch_multi_p(kh_ctx *ctx, MultiArgs a) {
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const int C = chunks_per_row(PREC, a.cols);
    const int cpl = C <= 2 * WAVE ? 1 : 2;  // short steps: a row in segments of one or two chunks per lane
    const int PB = padded_blocks(PREC, C, cpl);
    // token slots: the smallest of 2, 4, 8 that holds m, in as many launches
    // as the LDS stage needs (each launch streams the weights once).  A
    // workgroup may hold up to 160 KB of LDS on gfx950; a stage past half of
    // that leaves one workgroup per CU, and the grid is sized for that.
    constexpr size_t LDS_MAX = 160 * 1024;
    auto slots = [&](int left) {
        int T = left <= 2 ? 2 : left <= 4 ? 4 : 8;
        while (T > 2 && (size_t)T * PB * 40 > LDS_MAX) T /= 2;
        return T;
    };
    if ((size_t)slots(a.m) * PB * 40 > LDS_MAX) return fail(KH_DECLINED, "matmul: activation too wide for the LDS stage");
    const int per_cu = (size_t)slots(a.m) * PB * 40 > LDS_MAX / 2 ? 1 : 2;
    long long rows_total = 0;
    for (int i = 0; i < a.njobs; i++) rows_total += a.j[i].rows;
    int want = (int)((rows_total + WPB - 1) / WPB);
    if (want > per_cu * cu) want = per_cu * cu;
    // each job at least one workgroup, the rest in proportion to its rows
    int nwg = 0;
    for (int i = 0; i < a.njobs; i++) {
        int g = (int)((long long)want * a.j[i].rows / rows_total);
        if (g < 1) g = 1;
        a.j[i].wg0 = nwg;
        a.j[i].nwaves = g * WPB;
        nwg += g;
    }
    for (int t0 = 0; t0 < a.m;) {
        const int T = slots(a.m - t0);
        MultiArgs b = a;
        b.m = a.m - t0 < T ? a.m - t0 : T;
        if (a.xf) {
            b.xf = a.xf + (size_t)t0 * a.cols;
        } else {
            b.xq = a.xq + (size_t)t0 * a.cols;
            b.xs = a.xs + (size_t)t0 * (a.cols / BLOCK);
            b.xsum = a.xsum + (size_t)t0 * (a.cols / BLOCK);
        }
        for (int i = 0; i < a.njobs; i++) b.j[i].y = a.j[i].y + (size_t)t0 * a.j[i].rows;
        const size_t lds = (size_t)T * PB * 40;
        int rc = T == 2 ? launch_multi_t<PREC, 2>(ctx, b, cpl, nwg, lds)
                 : T == 4 ? launch_multi_t<PREC, 4>(ctx, b, cpl, nwg, lds)
                          : launch_multi_t<PREC, 8>(ctx, b, cpl, nwg, lds);
        if (rc) return rc;
        t0 += b.m;
    }
    return KH_OK;
}

int launch_gemv(kh_ctx *ctx, int precision, const GemvJob *jobs, int njobs) {
    // one launch per input kind present (a kernel stages one kind), in table order
    for (int i = 0; i < njobs; i++) {
        if (jobs[i].xf2 && jobs[i].norm_w) return fail(KH_EINVAL, "matvec: rms_norm and swiglu inputs do not combine");
        if (precision == KH_F32 && (jobs[i].xf2 || jobs[i].norm_w || !jobs[i].xf))
            return fail(KH_EINVAL, "matvec: the f32 GEMV takes its f32 input as it is");
    }
    for (int kind : {IN_F32, IN_NORM, IN_SWIGLU, IN_CODES}) {
        std::vector<GemvJob> js;
        for (int i = 0; i < njobs; i++)
            if (precision == KH_F32 || input_kind(jobs[i]) == kind) js.push_back(jobs[i]);
        for (int base = 0; base < (int)js.size(); base += MAX_JOBS) {
            JobTable tab{};
            tab.n = (int)js.size() - base < MAX_JOBS ? (int)js.size() - base : MAX_JOBS;
            int maxC = 0, maxCols = 0, rows_total = 0;
            bool dots = false;
            for (int i = 0; i < tab.n; i++) {
                tab.j[i] = js[base + i];
                int c = chunks_per_row(precision, tab.j[i].cols);
                maxC = c > maxC ? c : maxC;
                maxCols = tab.j[i].cols > maxCols ? tab.j[i].cols : maxCols;
                rows_total += tab.j[i].rows;
                dots = dots || tab.j[i].dots;
            }
            int rc;
            switch (precision) {
                case KH_Q8: rc = launch_prec<KH_Q8>(ctx, tab, maxC, maxCols, rows_total, dots, kind); break;
                case KH_Q4: rc = launch_prec<KH_Q4>(ctx, tab, maxC, maxCols, rows_total, dots, kind); break;
                case KH_Q4K: rc = launch_prec<KH_Q4K>(ctx, tab, maxC, maxCols, rows_total, dots, kind); break;
                case KH_F32: rc = launch_f32(ctx, tab); break;
                default: return fail(KH_EINVAL, "unknown precision");
            }
            if (rc != KH_OK) return rc;
        }
        if (precision == KH_F32) break;
    }
    return KH_OK;
}

int launch_gemv_route(kh_ctx *ctx, int precision, const GemvJob *jobs, int njobs, int route_job,
                      const RouteArgs &r) {
    if (njobs <= 0 || njobs > MAX_JOBS || route_job < 0 || route_job >= njobs)
        return fail(KH_EINVAL, "matvec: bad routed job table");
    if (r.n > MAX_EXPERTS || r.top_k > MAX_TOPK || r.n_group > MAX_GROUPS || jobs[route_job].rows != r.n)
        return fail(KH_DECLINED, "matvec: a router the fused routing does not take");
    if (precision != KH_Q8) return fail(KH_DECLINED, "matvec: routed launches are built for q8");
    JobTable tab{};
    tab.n = njobs;
    tab.route_job = route_job + 1;
    tab.route = r;
    int maxC = 0, maxCols = 0, rows_total = 0;
    for (int i = 0; i < njobs; i++) {
        tab.j[i] = jobs[i];
        if (input_kind(jobs[i]) != IN_F32 || jobs[i].dots) return fail(KH_DECLINED, "matvec: routed jobs take f32 x");
        const int c = chunks_per_row(precision, jobs[i].cols);
        maxC = c > maxC ? c : maxC;
        maxCols = jobs[i].cols > maxCols ? jobs[i].cols : maxCols;
        rows_total += jobs[i].rows;
    }
    return launch_prec<KH_Q8>(ctx, tab, maxC, maxCols, rows_total, false, IN_F32);
}

int launch_gemv_argmax(kh_ctx *ctx, int precision, const GemvJob &job, float *arg_v, int *arg_i, int *arg_n,
                       int cap, const GreedyTail *tail) {
    if (precision == KH_F32 || job.dots) return fail(KH_DECLINED, "matvec: the greedy epilogue is built for quantised weights");
    JobTable tab{};
    tab.n = 1;
    tab.j[0] = job;
    tab.arg_job = 1;
    tab.arg_cap = cap;
    tab.arg_v = arg_v;
    tab.arg_i = arg_i;
    tab.arg_n = arg_n;
    if (tail) tab.tail = *tail;
    const int maxC = chunks_per_row(precision, job.cols), kind = input_kind(job);
    switch (precision) {
        case KH_Q8: return launch_prec<KH_Q8>(ctx, tab, maxC, job.cols, job.rows, false, kind);
        case KH_Q4: return launch_prec<KH_Q4>(ctx, tab, maxC, job.cols, job.rows, false, kind);
        case KH_Q4K: return launch_prec<KH_Q4K>(ctx, tab, maxC, job.cols, job.rows, false, kind);
        default: return fail(KH_EINVAL, "unknown precision");
    }
}

int launch_gemv_multi_jobs(kh_ctx *ctx, int njobs, const kh_weight *const *w, const float *const *bias,
                           float *const *y, const int *accumulate, const QAct &x, size_t m, const float *xf) {
    if (m == 0) return KH_OK;
    // the matrix cores from mma_min_tokens() rows, and from two over a tall
    // matrix (a vocabulary head, 151936x896 at 2 rows: 32.3 against 35.9 us)
    size_t rows_total = 0;
    for (int i = 0; i < njobs && i < MULTI_JOBS; i++) rows_total += w[i]->rows;
    if (!xf && w[0]->precision != KH_F32 && (m >= mma_min_tokens() || (m >= 2 && rows_total >= 65536)))
        return launch_gemv_mma(ctx, njobs, w, bias, y, accumulate, x, m);
    if (njobs < 1 || njobs > MULTI_JOBS) return fail(KH_EINVAL, "matmul: one to three weights per launch");
    MultiArgs a{};
    a.xq = x.qs;
    a.xs = x.scales;
    a.xsum = x.sums;
    a.xf = xf;
    a.cols = (int)w[0]->cols;
    a.m = (int)m;
    a.njobs = njobs;
    for (int i = 0; i < njobs; i++) {
        if (w[i]->precision != w[0]->precision || w[i]->cols != w[0]->cols)
            return fail(KH_EINVAL, "matmul: weights of one launch share precision and width");
        if ((size_t)w[i]->rows * w[i]->cols >= 0xfff00000ull || m * w[i]->cols * (xf ? 4 : 1) >= 0xfff00000ull)
            return fail(KH_DECLINED, "matmul: operands of 4 GiB or more are not addressed here");
        a.j[i].w = w[i]->qs;
        a.j[i].ws = w[i]->scales;
        a.j[i].bias = bias ? bias[i] : nullptr;
        a.j[i].y = y[i];
        a.j[i].rows = (int)w[i]->rows;
        a.j[i].accumulate = accumulate ? accumulate[i] : 0;
    }
    switch (w[0]->precision) {
        case KH_Q8: return launch_multi_p<KH_Q8>(ctx, a);
        case KH_Q4: return launch_multi_p<KH_Q4>(ctx, a);
        case KH_Q4K: return launch_multi_p<KH_Q4K>(ctx, a);
        default: return fail(KH_EINVAL, "matmul: the multi-token GEMV takes quantised weights");
    }
}

int launch_gemv_multi(kh_ctx *ctx, const kh_weight *w, const QAct &x, size_t m, const float *bias, float *y) {
    return launch_gemv_multi_jobs(ctx, 1, &w, &bias, &y, nullptr, x, m);
}

bool multi_stages_f32(int precision, size_t m, size_t cols) {
    // Every workgroup quantises its token slots' rows (2, 4 or 8 slots); past
    // about 12K values that costs more than a quantising launch of its own
    // plus a stage of codes (measured over q8 and Q4_K weights of 896 to
    // 14336 columns at m = 2..8).
    // From mma_min_tokens() rows the matrix-core kernel takes the rows' codes.
    if (m >= mma_min_tokens()) return false;
    const size_t slots = m <= 2 ? 2 : m <= 4 ? 4 : 8;
    const int lim = env_int("KVAD_MULTI_STAGE_F32", 12288);  // tuning knob
    (void)precision;
    return slots * cols <= (size_t)lim;
}

size_t mma_min_tokens() { return (size_t)env_int("KVAD_MMA_MIN", 5); }  // tuning knob

bool matmul_takes_multi(size_t m, size_t rows, size_t cols) {
    const int forced = env_int("KVAD_MULTI_TOKENS", 0);  // tuning knob: the multi-token GEMV up to this many rows
    if (forced > 0) return m <= (size_t)forced;
    // Past eight rows the matrix-core kernel (16 rows a launch) beats the
    // GEMM only over narrow rows of a not-too-tall matrix; the GEMM's time is
    // nearly flat in m.  Measured (us): 4864x896 at 16 rows 10.1 against
    // 12.4; 896x896 7.9 / 12.1; 896x4864 18.1 / 12.0; 151936x896 (a
    // vocabulary head) 95.9 / 72.7, at 8 rows 49.7 / 72.0.
    return m <= (size_t)MULTI_TOKENS || (m <= 16 && cols <= 2048 && rows <= 16384);
}

bool gemv_pairs_fit(int precision, size_t cols) {
    if (precision == KH_F32 || env_int("KVAD_GEMV_PAIR", 1) == 0) return false;
    if (precision == KH_Q4K) return true;  // one or two chunks a lane
    return (chunks_per_row(precision, (int)cols) + WAVE - 1) / WAVE <= 4;
}

size_t fuse_max_cols(int precision) {
    static const size_t forced = [] {
        const char *e = getenv("KVAD_FUSE_MAX_COLS");
        return e && *e ? (size_t)atol(e) : (size_t)0;
    }();
    if (forced) return forced;
    return precision == KH_Q4K ? 16384 : 8192;
}

int launch_stream(kh_ctx *ctx, size_t n, const kh_weight *const *w, unsigned *sink) {
    StreamArgs a{};
    unsigned at = 0;
    for (size_t i = 0; i < n; i++) {
        const size_t qb = w[i]->precision == KH_Q8   ? w[i]->rows * w[i]->cols
                          : w[i]->precision == KH_Q4 ? w[i]->rows * w[i]->cols / 2
                          : w[i]->precision == KH_Q4K ? w[i]->rows * (w[i]->cols / QK_K) * Q4K_BYTES
                                                      : 4 * w[i]->rows * w[i]->cols;
        const size_t sb = w[i]->scales ? 4 * (w[i]->rows * w[i]->cols / BLOCK) : 0;
        for (int part = 0; part < 2; part++) {
            const size_t bytes = part ? sb : qb;
            if (!bytes) continue;
            if (a.n == STREAM_ARRAYS) return fail(KH_EINVAL, "stream: too many arrays");
            if (bytes % 16 || (size_t)at + bytes / 16 > 0x7fffffffu) return fail(KH_EINVAL, "stream: array size");
            at += (unsigned)(bytes / 16);
            a.p[a.n] = part ? (const void *)w[i]->scales : w[i]->qs;
            a.end[a.n++] = at;
        }
    }
    if (!a.n) return KH_OK;
    a.total = at;
    a.sink = sink;
    // the launch: `threads` a workgroup, about `wg` workgroups per CU, each
    // lane L loads (the fewest that keep within that many workgroups)
    const int cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const int wg = std::max(1, env_int("KVAD_STREAM_WG_PER_CU", 1));      // timing knob
    const int tk = env_int("KVAD_STREAM_THREADS", 256);                  // timing knob: 256, 512, 1024
    const int threads = tk == 1024 ? 1024 : tk == 512 ? 512 : 256;
    const int nt = env_int("KVAD_STREAM_NT", 0);                          // timing knob: non-temporal loads
    int L = 1;
    while (L < 16 && (at + (unsigned)(threads * L) - 1) / (unsigned)(threads * L) > (unsigned)(wg * cu)) L *= 2;
    const unsigned blocks = (at + (unsigned)(threads * L) - 1) / (unsigned)(threads * L);
#define KH_STREAM(LL)                                                                                      \
    case LL:                                                                                               \
        if (nt) hipLaunchKernelGGL((stream_kernel<LL, 2>), dim3(blocks), dim3(threads), 0, ctx->stream, a.p[0], \
                                   a.p[1], a.p[2], a.end[0], a.end[1], a.end[2], a.n, a.total, a.sink, a);    \
        else hipLaunchKernelGGL((stream_kernel<LL, 0>), dim3(blocks), dim3(threads), 0, ctx->stream, a.p[0],  \
                                a.p[1], a.p[2], a.end[0], a.end[1], a.end[2], a.n, a.total, a.sink, a);       \
        break;
    switch (L) {
        KH_STREAM(1) KH_STREAM(2) KH_STREAM(4) KH_STREAM(8)
        default: KH_STREAM(16)
    }
#undef KH_STREAM
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int launch_fill(kh_ctx *ctx, float *p, size_t n, float value) {
    if (n == 0) return KH_OK;
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, p, n, value);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int launch_dequant_row(kh_ctx *ctx, const kh_weight *w, size_t r, float *out) {
    hipLaunchKernelGGL(dequant_row_kernel, dim3((unsigned)((w->cols + 255) / 256)), dim3(256), 0, ctx->stream,
                       w->precision, (const void *)w->qs, (const float *)w->scales, w->cols, r,
                       (const int32_t *)nullptr, out);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

int launch_dequant_row_dev(kh_ctx *ctx, const kh_weight *w, const int32_t *r, float *out, size_t n) {
    if (n == 0) return KH_OK;
    if (n > 65535) return fail(KH_EINVAL, "rows: at most 65535 a launch");
    hipLaunchKernelGGL(dequant_row_kernel, dim3((unsigned)((w->cols + 255) / 256), (unsigned)n), dim3(256), 0,
                       ctx->stream, w->precision, (const void *)w->qs, (const float *)w->scales, w->cols, (size_t)0,
                       r, out);
    KH_HIP(hipGetLastError());
    return KH_OK;
}

}  // namespace kh
