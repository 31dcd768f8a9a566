// Internal declarations shared by the HIP translation units of libkvad_hip.
// Nothing here is part of the C ABI (include/kvad_hip.h is).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../include/kvad_hip.h"

namespace kh {

constexpr int BLOCK = 32;        // quant.rs:57
constexpr int QK_K = 256;        // Q4_K super-block
constexpr int Q4K_BYTES = 144;   // half d, half dmin, u8 scales[12], u8 qs[128]

// ---- errors -------------------------------------------------------------
void set_error(const std::string &msg);
int fail(int code, const std::string &msg);
int hip_fail(hipError_t e, const char *what);

#define KH_HIP(call)                                          \
    do {                                                      \
        hipError_t e_ = (call);                               \
        if (e_ != hipSuccess) return ::kh::hip_fail(e_, #call); \
    } while (0)

// A launch-shape tuning knob from the environment (dflt when unset).
inline int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

// ---- device workspace ---------------------------------------------------
// One growable device buffer per context, carved into named regions per
// call.  All work of a context runs on one stream, so reusing the same bytes
// call after call is ordered by the stream.
struct Workspace {
    void *ptr = nullptr;
    size_t bytes = 0;
};

// A packed activation: the QActivation/QActBatch arrays (quant.rs:1037-1066)
// for m rows of k values, resident in device memory.
struct QAct {
    int8_t *qs;      // [m * k]
    float *scales;   // [m * k / 32]
    int32_t *sums;   // [m * k / 32]
};

}  // namespace kh

struct kh_ctx {
    int device = 0;
    int cu_count = 0;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    std::recursive_mutex mu;
    kh::Workspace ws;        // per-call scratch (activations, partials)
    kh::Workspace io;        // staging for host-pointer calls
    kh::Workspace moe;       // mixture-of-experts intermediates
    kh::Workspace gemm;      // split-K partials
};

struct kh_weight {
    kh_ctx *ctx = nullptr;
    int precision = 0;  // KH_F32 / KH_Q8 / KH_Q4 / KH_Q4K
    size_t rows = 0, cols = 0;
    void *qs = nullptr;        // q8: int8[rows*cols]; q4: uint8[rows*cols/2]; q4k: blocks; f32: float[rows*cols]
    float *scales = nullptr;   // q8/q4: float[rows*cols/32]
    size_t bytes = 0;          // bytes held on the device
};

// A mixture-of-experts layer (model/ffn.rs:555-708): router settings and
// device tables of the experts' weights.  The weights are borrowed handles.
struct kh_moe {
    kh_ctx *ctx = nullptr;
    size_t n_experts = 0, top_k = 0, hidden = 0, inter = 0;
    int scoring = 0, select = 0, norm_topk = 0;
    size_t n_group = 1, topk_group = 1;
    float scale = 1.0f;
    float *bias = nullptr;                     // device [n_experts] or null
    const kh_weight *router = nullptr;
    std::vector<const kh_weight *> gate, up, down;
    const kh_weight *sgate = nullptr, *sup = nullptr, *sdown = nullptr;
    int precision = -1;                        // of every expert weight
    void **tab = nullptr;                      // device: [gate qs | up qs | down qs] x n_experts
    float **stab = nullptr;                    // device: the same for scales
    unsigned *arrivals = nullptr;              // device: router workgroups done this step (zero between steps)
    bool dirty = true;                         // tables need uploading
};

// A device-resident Llama-family decoder (crates/llm/src/model/llama.rs).
struct kh_llm {
    kh_ctx *ctx = nullptr;
    kh_llm_spec spec{};
    struct Layer {
        const kh_weight *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
        const kh_weight *gate = nullptr, *up = nullptr, *down = nullptr;
        float *attn_norm = nullptr, *mlp_norm = nullptr;     // device [n_embd]
        float *q_b = nullptr, *k_b = nullptr, *v_b = nullptr;  // device biases or null
        float *q_norm = nullptr, *k_norm = nullptr;          // device [head_dim] or null
    };
    std::vector<Layer> layers;
    const kh_weight *embed = nullptr, *head = nullptr;       // head null: tied to embed
    float *final_norm = nullptr;
    float *rope_cos = nullptr, *rope_sin = nullptr;          // [n_ctx, head_dim/2]
    std::vector<float *> kc, vc;                             // per layer [n_ctx, kv_dim]
    float *x = nullptr, *h = nullptr, *qkv = nullptr, *att = nullptr, *g = nullptr, *u = nullptr,
          *logits = nullptr;
    float *hsw = nullptr;                                    // swiglu(gate, up) of the step's SwiGLU pair
    kh::QAct hq{};
    int32_t *state = nullptr;                                // token, pos, step
    int32_t *token = nullptr, *pos = nullptr, *steps = nullptr;
    int32_t *out = nullptr;                                  // generated tokens
    float *arg_v = nullptr;                                  // argmax partials
    int *arg_i = nullptr;
    int *arg_n = nullptr;                                    // how many the head GEMV wrote
    unsigned *arrivals = nullptr;                            // head workgroups done this step (zero between steps)
    int out_cap = 0;
    void *attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    size_t len = 0;                                          // positions in the cache
    // one captured step per attention bucket, keyed by its launch maximum:
    // powers of two from 64 up to attn_short (attention as one split, no
    // merge launch), then n_ctx
    std::map<size_t, hipGraphExec_t> graphs;
    size_t attn_short = 0;                                   // attend_single_max, at most n_ctx
    size_t attn_max = 0;                                     // the launch maximum of the step being issued
    // Session::park / resume (model/mod.rs:889-897): caches handed out and
    // not yet taken back or freed, and freed ones kept for the next park
    std::set<kh_llm_parked *> parked;
    std::vector<std::pair<std::vector<float *>, std::vector<float *>>> spare;
    // forward_each's buffers for rows_cap rows, one allocation laid out by
    // session.hip, and the host copy of the table it uploads per call
    void *rows_buf = nullptr;
    size_t rows_cap = 0;
    std::vector<char> rows_host;
    std::map<std::pair<size_t, size_t>, hipGraphExec_t> rows_graphs;  // the pass for n rows, per (n, bucket)
    // a prompt read in passes of up to `chunk` tokens (Session::prefill_pass),
    // each pass of n > 1 rows captured per (n, attention bucket) in the same
    // rows buffer
    size_t chunk = 0;
    std::map<std::pair<size_t, size_t>, hipGraphExec_t> pass_graphs;
    void *pass_buf = nullptr;   // the pass's rows, for pass_cap rows
    size_t pass_cap = 0;
    kh::Workspace pass_ws;      // the pass's attention partials
};

// A conversation's cache set aside (Session::park, model/mod.rs:889-893): per
// layer [n_ctx, kv_dim] keys and values, and the positions held.
struct kh_llm_parked {
    kh_llm *owner = nullptr;  // null once the session is freed
    int device = 0;
    std::vector<float *> k, v;
    size_t len = 0;
};

struct kh_kv {
    kh_ctx *ctx = nullptr;
    size_t n_layer = 0, k_dim = 0, v_dim = 0;
    size_t capacity = 0;              // positions allocated per layer
    size_t len = 0;                   // KvCache::len (mod.rs:623)
    std::vector<float *> k, v;        // per layer, [capacity, dim]
    std::vector<size_t> rows;         // positions pushed per layer
};

namespace kh {

// Grows `w` to at least `bytes` (synchronising the stream before freeing).
int ensure(kh_ctx *ctx, Workspace &w, size_t bytes);

// ---- launchers (each defined in the .hip file that holds its kernels) ----
// Activation quantiser: m rows of k floats -> QAct.  k % 32 == 0.
int launch_qact(kh_ctx *ctx, const float *x, size_t m, size_t k, const QAct &out);
int launch_quant_check(kh_ctx *ctx, unsigned long long *counts);  // counts[3], device, zeroed

// One GEMV job: y[rows] = x W^T (+bias) for a quantised or f32 weight.
struct GemvJob {
    const void *w;          // weight bytes (qs / blocks / f32)
    const float *ws;        // q8/q4 scales (null for q4k/f32)
    const int8_t *xq;       // quantised activation (q8/q4/q4k)
    const float *xs;        // activation scales
    const int32_t *xsum;    // activation block sums
    const float *xf;        // f32 activation: quantised in the kernel (or read
                            // as is by f32 weights); null when xq.. are given
    const float *bias;      // or null
    float *y;
    int32_t *dots;          // optional: pass-1 integers, [rows * cols/32]
    // Expert indirection (MoE decode): when wtab is set the weight is
    // wtab[*sel] (scales wstab[*sel]), read from device memory by the kernel.
    const void *const *wtab;
    const float *const *wstab;
    const int32_t *sel;
    const float *xf2;       // with xf: the staged activation is swiglu(xf, xf2)
    int accumulate;         // y[r] = y[r] + (x W^T + bias)[r]: the residual add
    const float *norm_w;    // with xf: the staged activation is rms_norm(xf, norm_w, norm_eps)
    float norm_eps;
    int rows;
    int cols;
    int wave0;              // set by the launcher: first workgroup of the job
    int nwaves;             // set by the launcher: waves working on the job
    // SwiGLU pairs (the decode step's gate and up, ffn.rs:370-386): when w2
    // is set, the job's rows are gate row i (w, ws) and up row i (w2, ws2)
    // interleaved, rows = 2 * n_ff; gate row i goes to y[i], up row i to
    // y2[i] and swiglu(gate, up) (tensor.rs:344-350) to h[i].  No bias, no
    // accumulate; the job is its launch's only one.
    const void *w2;
    const float *ws2;
    float *y2, *h;
};
// Whether a SwiGLU-pair job takes `precision` weights `cols` wide (the
// launch needs an even number of rows a step).
bool gemv_pairs_fit(int precision, size_t cols);

// Weight::matvec_bt_dequant (quant.rs:522-589, dequant.hip): y = x W^T
// (+ bias) with the weights unpacked to f32 and x used as it is, for q8, q4
// and Q4_K weights; one launch.
int launch_gemv_dequant(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y);
// Whether KVAD_DEQUANT asks for it (quant.rs:608-610: "1" or "true").
bool dequant_selected();

// Widest rows whose GEMV quantises its f32 input itself (each workgroup
// stages it in LDS); wider inputs are quantised once in a launch of their own.
size_t fuse_max_cols(int precision);

// Runs every job in one launch per input kind (all jobs share `precision`).
int launch_gemv(kh_ctx *ctx, int precision, const GemvJob *jobs, int njobs);
struct RouteArgs;
// One launch of `jobs` (f32 inputs, q8) whose job route_job is a router:
// its one workgroup computes the token's logits and routes them (r.logits
// unused); KH_DECLINED where no such kernel is built for the launch's shape.
int launch_gemv_route(kh_ctx *ctx, int precision, const GemvJob *jobs, int njobs, int route_job, const RouteArgs &r);
// A decode step's end folded into the head GEMV: the last of its workgroups
// to finish takes the best of their choices against row 0 (the first of
// equal maxima wins; sampler.rs:217-226), makes it the next token, advances
// the position, records the step (out[step] while step < out_cap) and
// writes the token's embedding row to x.
struct GreedyTail {
    unsigned *arrivals;  // device: head workgroups done this step (zero between steps)
    int32_t *token, *pos, *step, *out;
    int out_cap;
    int prec;  // the embedding's
    const void *qs;
    const float *scales;
    size_t cols;
    float *x;
};
// One GEMV whose workgroups also keep the greedy choice over their rows
// r >= 1 (workgroup g: arg_v[g], arg_i[g]; their count to *arg_n), and with
// `tail` set end the step as GreedyTail says; KH_DECLINED for f32 weights or
// more than `cap` workgroups.
int launch_gemv_argmax(kh_ctx *ctx, int precision, const GemvJob &job, float *arg_v, int *arg_i, int *arg_n,
                       int cap, const GreedyTail *tail = nullptr);

// y[m, rows] = x W^T (+bias) for a few quantised token rows (m small): the
// weights stream once for all of them.  x holds the rows' codes.
constexpr int MULTI_TOKENS = 8;  // token slots of one VALU multi-token launch
// Whether m token rows against a rows x cols weight take the multi-token
// GEMV (else the GEMM): kh_matmul, and the session's single projections.
bool matmul_takes_multi(size_t m, size_t rows, size_t cols);
int launch_gemv_multi(kh_ctx *ctx, const kh_weight *w, const QAct &x, size_t m, const float *bias, float *y);
// The same for up to MULTI_JOBS weights of one precision and width over the
// same rows of codes, in one launch: y[i] (+)= x W_i^T (+ bias[i]), adding
// into y[i] where accumulate[i] is set (accumulate and bias may be null).
// With xf set, the rows are f32 ([m][cols]) and every workgroup quantises
// them as it stages them (the same codes as launch_qact); x is then unused.
constexpr int MULTI_JOBS = 3;
// The second and third jobs' first workgroups of a multi-token launch as one
// 16-bit-pair word (0xffff: no such job), passed as a leading kernel
// argument, which the build preloads into a scalar register: a workgroup
// finds its job without a load.
inline unsigned multi_firsts(int njobs, int g1, int g2) {
    const unsigned a = njobs > 1 && g1 < 0xffff ? (unsigned)g1 : 0xffffu;
    const unsigned b = njobs > 2 && g2 < 0xffff ? (unsigned)g2 : 0xffffu;
    return a | b << 16;
}
// Whether the multi-token GEMV should stage m f32 rows of `cols` itself
// (quantising them in every workgroup) rather than read codes quantised once
// by a launch of their own: only while the stage is small.
bool multi_stages_f32(int precision, size_t m, size_t cols);
// Token rows from which the multi-token GEMV runs on the matrix cores
// (launch_gemv_mma) when it is given codes.
size_t mma_min_tokens();
// The multi-token GEMV on the matrix cores (gemv_mma.hip): the same
// contract as launch_gemv_multi_jobs over codes, 16 token rows a launch.
int launch_gemv_mma(kh_ctx *ctx, int njobs, const kh_weight *const *w, const float *const *bias, float *const *y,
                    const int *accumulate, const QAct &x, size_t m);
int launch_gemv_multi_jobs(kh_ctx *ctx, int njobs, const kh_weight *const *w, const float *const *bias,
                           float *const *y, const int *accumulate, const QAct &x, size_t m,
                           const float *xf = nullptr);

// Batched prefill y[m, rows] = xs[m, cols] W^T (+bias), m > 1 (device pointers).
int launch_matmul(kh_ctx *ctx, const kh_weight *w, const float *xs, size_t m, const float *bias, float *y,
                  int accumulate = 0);
// The same over rows already quantised (QActBatch form), quantised weights
// only; with accumulate, y += the product.
int launch_matmul_q(kh_ctx *ctx, const kh_weight *w, const QAct &q, size_t m, const float *bias, float *y,
                    int accumulate = 0);

// GEMM over activations already quantised (QActBatch form), optionally
// grouped by expert: with `tiles` set, workgroup row y of the grid takes tile
// tiles[1 + 3y .. 3 + 3y] = (expert, first row, rows) of tiles[0] tiles, its
// weight is wtab[expert], and activation row r of the tile is gather[r]
// (or r).  Output row r is y + r * N.
struct GemmArgs {
    const void *w;          // q8 int8 / q4 packed / Q4_K blocks / f32 [N, K]
    const float *ws;        // q8/q4 block scales [N, K/32]
    const int8_t *xq;       // quantised activations [M, K]
    const float *xs;        // activation block scales [M, K/32]
    const int32_t *xsum;    // activation block sums [M, K/32] (Q4_K)
    const float *xf;        // f32 activations [M, K] (f32 GEMM)
    const float *bias;      // [N] or null
    float *y;               // [M, N]
    int accumulate;         // y += x W^T (+ bias): the residual add
    int M, N, K;
    const int32_t *tiles;
    const int32_t *gather;
    const void *const *wtab;
    const float *const *wstab;
    // split-K (ungrouped launches): ksplit > 1 splits the k-stages over grid
    // z; split z writes its tile to part[z][M][N] and a second launch adds
    // the splits in order, then bias and residual
    int ksplit;
    float *part;
    // a second weight of the same shape over the same activations (gate and
    // up): when y2 is set the grid holds both weights' row tiles, the first
    // weight's then the second's, and the second writes y2 (split-K partials
    // of the second take the plane after the first's)
    const void *w2;
    const float *ws2;
    const void *const *wtab2;
    const float *const *wstab2;
    float *y2;
};
// tile_n: weight rows per tile (128, or 64 with 64-token tiles, ungrouped)
int launch_gemm_q(kh_ctx *ctx, int precision, const GemmArgs &a, int max_tiles, int tile_m, int tile_n = 128);
// Allocates the split-K workspace now (a GEMM captured into a graph splits
// only when it was allocated before the capture).
int gemm_split_reserve(kh_ctx *ctx);
// Sets a's split-K fields for an ungrouped launch of tile_m-token tiles when
// splitting its k-stages pays (ksplit 0: no split).
int plan_split(kh_ctx *ctx, GemmArgs &a, int tile_m, int tile_n = 128);
// Tokens per tile (returned) and weight rows per tile (*tile_n) for an
// ungrouped M x N launch of the int8 GEMM.
int gemm_tiles(kh_ctx *ctx, int M, int N, int *tile_n);

// Operator bodies on device pointers (abi.hip), for the layers built on them.
int matvec_device(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y, int32_t *dots);
int matvec_many_device(kh_ctx *ctx, size_t n, const kh_weight *const *w, const float *const *x, float *const *y);
int matmul_device(kh_ctx *ctx, const kh_weight *w, const float *xs, size_t m, const float *bias, float *y);
// QActBatch::new of rms_norm(x) * w (gemv.hip): m rows of n values (n % 32 ==
// 0), the normed rows also into h when h is set.
int launch_norm_qact(kh_ctx *ctx, const float *x, const float *w, size_t m, size_t n, float eps, float *h,
                     const QAct &out);
// QActBatch::new of swiglu(g, u) (gemv.hip): m rows of k values.
int launch_swiglu_qact(kh_ctx *ctx, const float *g, const float *u, size_t m, size_t k, const QAct &out);
// Moe::run on device pointers, and Router::route alone (moe.hip).
int moe_run_device(kh_ctx *ctx, kh_moe *moe, const float *hs, size_t m, float *out);
// A debugging aid: after a MoE run of m tokens, its intermediates per token
// and pick (picks in expert order, unused ones zero), copied to the host.
// Any pointer may be null.
struct MoePicks {
    float *logits;                    // [m][n_experts]
    int32_t *count;                   // [m]
    int32_t *experts;                 // [m][top_k]
    float *weights;                   // [m][top_k]
    float *gate, *up;                 // [m][top_k][inter]
    int8_t *hidden_qs;                // [m][top_k][inter] (m > 1 only)
    float *hidden_scales;             // [m][top_k][inter / 32]
    float *out;                       // [m][top_k][hidden]
    float *shared_gate, *shared_up;   // [m][shared width]
    float *shared_out;                // [m][hidden]
};
int moe_picks(kh_ctx *ctx, const kh_moe *moe, size_t m, const MoePicks &o);
int route_device(kh_ctx *ctx, const kh_moe *moe, const float *logits, size_t m, int32_t *experts, float *weights,
                 int32_t *count);

// ---- mixture of experts (moe.hip) ----
// Router::route for m tokens (logits [m, n]): experts/weights [m, top_k] in
// pick order, count [m]; with `sorted` set, the picks of each token are
// reordered by expert index (the order mix() adds them in).
struct RouteArgs {
    const float *logits;
    const float *bias;      // [n] or null
    int n, top_k, scoring, select, n_group, topk_group, norm_topk, always_scale;
    float scale;
    int32_t *experts;
    float *weights;
    int32_t *count;
    int32_t *sorted_experts;  // optional, [m, top_k]
    float *sorted_weights;
    // Fused into the router's GEMV (launch_gemv_route): with `arrivals` set,
    // the router's rows are spread over `groups` workgroups and the last to
    // finish routes; without, one workgroup computes them all and routes.
    unsigned *arrivals;
    int groups;
};
int launch_route(kh_ctx *ctx, const RouteArgs &r, int m);

// Split decode attention over one layer's cache, device pointers.
int launch_attend(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const float *k,
                  const float *v, size_t kv_stride_k, size_t kv_stride_v, size_t n_positions, float *out);

// Weight::quantize on device f32 data into qs/scales (scales unused for Q4_K).
int launch_quantize(kh_ctx *ctx, const float *w, size_t rows, size_t cols, int precision, void *qs, float *scales);

// Small helpers.
int launch_fill(kh_ctx *ctx, float *p, size_t n, float value);
// The weights' bytes read once by a streaming kernel (timing aid); each
// workgroup writes one word of sink [STREAM_SINK].
constexpr unsigned STREAM_SINK = 4096;
int launch_stream(kh_ctx *ctx, size_t n, const kh_weight *const *w, unsigned *sink);
int launch_dequant_row(kh_ctx *ctx, const kh_weight *w, size_t r, float *out);
// The same with the row indices read from device memory (an embedding
// lookup): rows r[0..n) into out [n][cols].
int launch_dequant_row_dev(kh_ctx *ctx, const kh_weight *w, const int32_t *r, float *out, size_t n = 1);
// tensor::rms_norm over m rows of n (glue.hip).
int launch_rms_norm(kh_ctx *ctx, const float *x, const float *w, size_t m, size_t n, float eps, float *out);
// gate = silu(gate) * up over n floats (glue.hip).
int launch_swiglu(kh_ctx *ctx, float *gate, const float *up, size_t n);
// A row of a batched attention launch: its caches and its length.
struct AttnRow {
    float *k, *v;
    int L;
};
// RoPE and the cache push of the new position fused into the attention
// (the session's step): the new token's key and value unrotated (kraw, vraw;
// raw_stride floats apart per batched row), the tables [max_pos][hd/2],
// optional per-head norms (Qwen3) and the pairing.  The query passed to the
// launch is unrotated too.
struct AttnRope {
    const float *kraw, *vraw;
    const float *cos_t, *sin_t, *q_norm, *k_norm;
    float eps;
    int interleaved;
    size_t raw_stride;
};

// Attention whose length is read from device memory: n_positions = *len_dev
// (+1 when plus_one), at most max_positions; partials in `ws` (attend_ws_bytes).
int launch_attend_devlen(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const float *k,
                         const float *v, size_t kv_stride_k, size_t kv_stride_v, const int32_t *len_dev, int plus_one,
                         size_t max_positions, float *out, void *ws, size_t ws_bytes,
                         const AttnRope *rope = nullptr);
size_t attend_ws_bytes(int n_head, int n_kv_head, int head_dim, size_t max_positions);
// The longest sequence the launches above take as one split (no partials,
// no merge launch); 0 when none.
size_t attend_single_max(int head_dim);
// Attention with its partials in the library's static per-device scratch
// array (attend.hip): no allocation.  scratch_init(device), with that device
// current, looks up the array's device address once per device (kh_init
// calls it); scratch_bytes() is the array's size.
int scratch_init(int device);
size_t scratch_bytes();
int launch_attend_noalloc(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const float *k,
                          const float *v, size_t kstride, size_t vstride, size_t n_positions, float *out);
// Attention of nb rows at once, each over its own cache (forward_each,
// llama.rs:258-271): row z's query is q + z * n_head * head_dim, its output
// out + z * n_head * head_dim, its keys and values rows[z].k / .v (strides
// kstride / vstride) over rows[z].L <= max_positions positions.  `rows` is in
// device memory; partials in `ws` (attend_rows_ws_bytes).
int launch_attend_rows(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const AttnRow *rows,
                       int nb, size_t kstride, size_t vstride, size_t max_positions, float *out, void *ws,
                       size_t ws_bytes, const AttnRope *rope = nullptr);
size_t attend_rows_ws_bytes(int n_head, int head_dim, size_t max_positions, size_t nb);
// The partials launch_attend_rows needs for nb rows of at most max_positions
// on this context (the split it would pick), in bytes; 0 when it would refuse.
size_t attend_rows_need_bytes(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, size_t max_positions, size_t nb);
// Attention of one sequence's pass (Rows::Following): n rows of q (rotated)
// over one cache (rows[0]'s), row i over positions 0 .. rows[i].L - 1, every
// row's whole sequence in one wave (no partials), at most max_positions.
// attend_pass_fits says whether the launch takes the shape (head_dim 64 or
// 128, the cache addressed in 32 bits) and is not switched off
// (KVAD_PASS_ATTN=0 keeps a pass on launch_attend_rows).
bool attend_pass_fits(int head_dim, size_t kstride, size_t vstride, size_t max_positions);
int launch_attend_pass(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const AttnRow *rows,
                       int n, size_t kstride, size_t vstride, size_t max_positions, float *out);
// The rows of one sequence's pass (Rows::Following): queries q [nb][n_head][hd]
// normed and rotated in place, keys k [nb][n_kv][hd] normed, rotated and
// written with the values v into each row's cache at rows[i].L - 1.
int launch_rope_push_rows(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, float *q, const float *k,
                          const float *v, const AttnRow *rows, int nb, size_t kstride, size_t vstride,
                          const AttnRope &rope);

// Absorbed latent attention (model/deepseek.rs:553-591): out[n_head][512] =
// softmax over positions of (q_lat . c_t + q_pe . pe_t) * scale, times c_t.
int launch_mla(kh_ctx *ctx, int n_head, const float *q_lat, const float *q_pe, const float *c, const float *pe,
               size_t cstride, size_t pestride, size_t n_positions, float scale, float *out);

}  // namespace kh
