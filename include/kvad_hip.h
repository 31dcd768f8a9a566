/*
 * kvad_hip.h -- C ABI of libkvad_hip, the MI355X (gfx950) implementation of
 * kvad's quantised matmul and decode attention.
 *
 * Every entry point replaces one operator of the reference crate
 * (bisand/kvad, crates/llm) and is written so that the Rust side can bind it
 * with a plain `extern "C"` block: plain C types, pointers and sizes, no
 * ownership crossing the boundary except through the opaque handles below.
 *
 * Conventions (mirroring the reference):
 *   - Every function returns an int status: KH_OK (0), KH_DECLINED (1: the
 *     caller should run its CPU kernel, as `matvec_many` returning None does,
 *     quant.rs:626-633), or a negative error.  kh_last_error() gives the
 *     message for the calling thread.  Nothing aborts.
 *   - Functions taking host pointers are synchronous: they copy inputs in,
 *     run, copy results out and return.  `_dev` variants take device
 *     pointers and are asynchronous on the context's stream.
 *   - Weights are uploaded from borrowed host arrays in kvad's own layout
 *     (quant.rs:121-127, qcache.rs:30-40): the handle owns the device copy.
 *   - Calls on one context are serialised by an internal mutex; separate
 *     contexts may be used from separate threads.
 */
#ifndef KVAD_HIP_H
#define KVAD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KH_OK 0
#define KH_DECLINED 1
#define KH_EINVAL (-1)
#define KH_EHIP (-2)
#define KH_ENOMEM (-3)

/* Precision of a weight: quant.rs:59-64 (F32, Q8, Q4) plus GGML's Q4_K,
 * whose block layout is gpu/src/mpp.rs:241-251. */
#define KH_F32 0
#define KH_Q8 1
#define KH_Q4 2
#define KH_Q4K 3

typedef struct kh_ctx kh_ctx;
typedef struct kh_weight kh_weight;
typedef struct kh_kv kh_kv;

/* The calling thread's last error message; library-owned, valid until the
 * thread's next call.  House style of apps/phone/core/kvad_core.h:27. */
const char *kh_last_error(void);

/* Library version string.  Static; never freed (kvad_core.h:26-27). */
const char *kh_version(void);

/* ---- context ---------------------------------------------------------- */

/* A device and a stream: the per-session state CpuSession keeps as its rayon
 * pool (model/mod.rs:979-1072). */
int kh_init(int device, kh_ctx **out);
/* Frees the context.  Every weight, cache, MoE layer, session and parked
 * conversation made on it must be freed first: their frees lock the
 * context. */
int kh_free(kh_ctx *ctx);
/* Launch on `hip_stream` (a hipStream_t) instead of the context's own; NULL
 * restores the own stream.  The caller keeps ownership of the stream. */
int kh_set_stream(kh_ctx *ctx, void *hip_stream);
int kh_synchronize(kh_ctx *ctx);
/* Grow the context's device scratch to `bytes` up front, so that later calls
 * do not allocate. */
int kh_reserve(kh_ctx *ctx, size_t bytes);

/* ---- weights ---------------------------------------------------------- */

/* Weight::from_q8 (quant.rs:287-290): scales f32[rows*cols/32], qs
 * i8[rows*cols], row-major; cols % 32 == 0 (quant.rs:131-142). */
int kh_weight_q8(kh_ctx *ctx, size_t rows, size_t cols, const float *scales, const int8_t *qs,
                 kh_weight **out);
/* Weight::from_q4 (quant.rs:292-295): scales f32[rows*cols/32], qs
 * u8[rows*cols/2]; byte k of a block holds weight k (low nibble) and k+16
 * (high nibble), bias 8 (quant.rs:258-274). */
int kh_weight_q4(kh_ctx *ctx, size_t rows, size_t cols, const float *scales, const uint8_t *qs,
                 kh_weight **out);
/* GGML Q4_K blocks, 144 bytes per 256 weights, rows of cols/256 blocks
 * (gpu/src/mpp.rs:241-251); cols % 256 == 0. */
int kh_weight_q4k(kh_ctx *ctx, size_t rows, size_t cols, const uint8_t *blocks, kh_weight **out);
/* Weight::from_f32 (quant.rs:331-333): data f32[rows*cols]. */
int kh_weight_f32(kh_ctx *ctx, size_t rows, size_t cols, const float *data, kh_weight **out);
/* Weight::quantize (quant.rs:209-281) on the device, from f32 data
 * [rows, cols]: precision KH_Q8 or KH_Q4 as the reference quantises, KH_Q4K
 * with this library's packing of GGML's block (any valid packing; the GEMV
 * reads whatever bytes it is given).  Bit-identical to the CPU quantiser.
 * KH_F32, and any width that does not divide into blocks, keeps the data as
 * an f32 weight (quant.rs:211-213). 
 * `data` is a host pointer; the _dev form takes a device pointer. */
int kh_weight_quantize(kh_ctx *ctx, size_t rows, size_t cols, const float *data, int precision, kh_weight **out);
int kh_weight_quantize_dev(kh_ctx *ctx, size_t rows, size_t cols, const float *data, int precision,
                           kh_weight **out);
/* Weight::parts (quant.rs:336-342): copy the stored arrays back to the host.
 * qs receives rows*cols (q8), rows*cols/2 (q4), rows*cols/256*144 (Q4_K) or
 * 4*rows*cols (f32) bytes; scales rows*cols/32 floats (q8/q4; else unused). */
int kh_weight_parts(const kh_weight *w, void *qs, float *scales);
int kh_weight_free(kh_weight *w);
/* rows, cols, precision and device bytes (Weight::bytes, quant.rs:365-371). */
int kh_weight_info(const kh_weight *w, size_t *rows, size_t *cols, int *precision, size_t *bytes);
/* Weight::row (quant.rs:374-402): row r dequantised to f32 (the embedding
 * lookup).  Q4_K rows decode as mpp.rs:304-315. */
int kh_weight_row(kh_ctx *ctx, const kh_weight *w, size_t r, float *out);

/* ---- GEMV / GEMM ------------------------------------------------------ */

/* Weight::matvec_bt (quant.rs:481-512): y[rows] = x[cols] W^T (+ bias).
 * Quantised weights quantise x per 32-block first (QActivation::new,
 * quant.rs:1044-1066).  bias may be NULL. */
int kh_matvec(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y);
int kh_matvec_dev(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y);

/* Weight::matvec_bt_dequant (quant.rs:522-589): the same product with each
 * weight unpacked to f32 and x used as it is, unquantised -- the baseline the
 * reference keeps beside its integer path and selects with KVAD_DEQUANT=1
 * (quant.rs:592-610).  With KVAD_DEQUANT set to "1" or "true", kh_matvec and
 * kh_matvec_dev (and kh_matmul at m == 1) run this kernel too, and
 * kh_matvec_many declines, as matvec_many returns None.  q8, q4 and Q4_K
 * weights (Q4_K as mpp.rs:304-315 decodes it); f32 weights are KH_EINVAL. */
int kh_matvec_dequant(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y);
int kh_matvec_dequant_dev(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y);

/* quant::matvec_many (quant.rs:628-671): n GEMVs in one launch, each result
 * bit-identical to kh_matvec on the same job.  Returns KH_DECLINED when a
 * weight is f32 or x's length does not match, as the reference returns None. */
int kh_matvec_many(kh_ctx *ctx, size_t n, const kh_weight *const *w, const float *const *x,
                   float *const *y);
int kh_matvec_many_dev(kh_ctx *ctx, size_t n, const kh_weight *const *w, const float *const *x,
                       float *const *y);

/* Weight::matmul_bt (quant.rs:751-858): y[m, rows] = xs[m, cols] W^T (+ bias);
 * m == 1 is kh_matvec. */
int kh_matmul(kh_ctx *ctx, const kh_weight *w, const float *xs, size_t m, const float *bias, float *y);
int kh_matmul_dev(kh_ctx *ctx, const kh_weight *w, const float *xs, size_t m, const float *bias, float *y);

/* QActBatch::new (quant.rs:693-714) on the device: m rows of n floats (n %
 * 32 == 0) -> qs i8[m*n], scales f32[m*n/32], sums i32[m*n/32].  The
 * activation form the GEMV and GEMM kernels read; a producer kernel that
 * already holds it can skip kh_matvec's own quantisation step. */
int kh_qact_dev(kh_ctx *ctx, const float *x, size_t m, size_t n, int8_t *qs, float *scales, int32_t *sums);
/* Weight::qrow over every row (quant.rs:410-452) for an activation already
 * quantised by kh_qact_dev: the GEMV kernel alone.  Not for f32 weights. */
int kh_matvec_q_dev(kh_ctx *ctx, const kh_weight *w, const int8_t *qs, const float *scales, const int32_t *sums,
                    const float *bias, float *y);

/* Parity hooks.  Pass-1 integers of the GEMV kernel that kh_matvec runs
 * (quant.rs:426-440): dots[rows * cols/32].  For Q4_K, dots are
 * sum(q * xq) over each 32-wide sub-block with q the unsigned 4-bit code. */
int kh_debug_block_dots(kh_ctx *ctx, const kh_weight *w, const float *x, int32_t *dots);
/* QActivation::new on the device: qs[n], scales[n/32], sums[n/32]. */
int kh_debug_qact(kh_ctx *ctx, const float *x, size_t n, int8_t *qs, float *scales, int32_t *sums);
/* Self-check (no counterpart in the reference): the device arithmetic of
 * QActivation::new (quant.rs:1051-1059) over every float.  counts[0] and
 * counts[1]: scales and inverses, for each finite amax >= 0, that differ from
 * the IEEE quotients amax / 127 and 1 / scale; counts[2]: codes, for each of
 * the 2^32 patterns t, that differ from t.round().clamp(-127.0, 127.0) as i8.
 * All three are 0 on a correct build.  Synchronous. */
int kh_debug_quant_check(kh_ctx *ctx, uint64_t *counts);
/* Timing aid (no counterpart in the reference): one launch that reads every
 * byte of up to four weights once (codes and scales) with 16-byte loads and
 * no arithmetic, each workgroup writing one word of the device array
 * sink[4096]; asynchronous on the context's stream.  Set beside the GEMV's
 * launches over the same weights it gives the HBM ceiling of that launch
 * structure. */
int kh_debug_stream_dev(kh_ctx *ctx, size_t n, const kh_weight *const *w, uint32_t *sink);

/* ---- KV cache and attention ------------------------------------------- */

/* KvCache (model/mod.rs:612-749), device-resident: per layer an append-only
 * [capacity, k_dim] key and [capacity, v_dim] value array; grows by doubling
 * (the design of gpu/src/common.rs:547-700). */
int kh_kv_new(kh_ctx *ctx, size_t n_layer, size_t k_dim, size_t v_dim, size_t capacity, kh_kv **out);
int kh_kv_free(kh_kv *kv);
/* KvCache::push (mod.rs:666-669): m rows appended to `layer`. */
int kh_kv_push(kh_kv *kv, size_t layer, const float *k, const float *v, size_t m);
int kh_kv_push_dev(kh_kv *kv, size_t layer, const float *k, const float *v, size_t m);
/* KvCache::len (mod.rs:623), read and set as the model advances it. */
int kh_kv_len(const kh_kv *kv, size_t *len);
int kh_kv_set_len(kh_kv *kv, size_t len);
/* KvCache::truncate (mod.rs:709-725): keep the first `len` positions of
 * every layer; *kept receives the length actually kept. */
int kh_kv_truncate(kh_kv *kv, size_t len, size_t *kept);
/* KvCache::clear (mod.rs:727-738). */
int kh_kv_clear(kh_kv *kv);
/* KvCache::keys / values (mod.rs:671-677): copy the pushed rows of a layer
 * to the host (rows * dim floats); *rows receives the row count. */
int kh_kv_keys(const kh_kv *kv, size_t layer, float *out, size_t *rows);
int kh_kv_values(const kh_kv *kv, size_t layer, float *out, size_t *rows);
/* Device pointers of a layer's arrays (valid until the next push that grows). */
int kh_kv_layer_ptrs(const kh_kv *kv, size_t layer, float **k, float **v);

/* model::attend (model/mod.rs:769-819): GQA decode attention of one query
 * (n_head * head_dim floats) over the first n_positions rows of `layer`;
 * out is n_head * head_dim floats.  Same weights as the reference,
 * including its skip of weights below 1e-8 (mod.rs:807). */
int kh_attend(kh_ctx *ctx, const kh_kv *kv, size_t layer, size_t n_head, size_t n_kv_head,
              size_t head_dim, const float *q, size_t n_positions, float *out);
/* The same over raw device arrays: k and v rows are n_kv_head*head_dim wide. */
int kh_attend_dev(kh_ctx *ctx, size_t n_head, size_t n_kv_head, size_t head_dim, const float *q,
                  const float *k, const float *v, size_t n_positions, float *out);

/* kh_attend_dev without allocating: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): the same kernels,
 * with the split partials in a static device array of
 * kh_noalloc_scratch_bytes() bytes (8 MiB) that each GPU holds from library
 * load until the process ends; kh_init looks up its address once per device.
 * A call whose partials need more (long contexts at many heads: about 2.3 MB
 * at Qwen2.5-0.5B geometry and 32768 positions) is KH_EINVAL with the size in
 * kh_last_error().  Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams or threads) race; calls on one stream
 * are ordered. */
int kh_attend_dev_noalloc(kh_ctx *ctx, size_t n_head, size_t n_kv_head, size_t head_dim, const float *q,
                          const float *k, const float *v, size_t n_positions, float *out);
size_t kh_noalloc_scratch_bytes(void);

/* Latent attention, absorbed (model/deepseek.rs:553-591), one token: head h
 * scores cached position t as (q_lat_h . c_t + q_pe_h . pe_t) * scale,
 * softmax over the positions, and returns the attended latent
 * out[h] = sum_t w_t c_t (512 wide; weights below 1e-8 dropped, mod.rs:807's
 * rule as deepseek.rs:576-579 applies it).  The uk / uv projections around
 * it are matvecs.  The cache is the reference's: keys are the rotated pe rows
 * (64 wide), values the normed latents c (512 wide), KvCache::push(layer,
 * k_pe, c) at deepseek.rs:540-547.  q_lat [n_head*512], q_pe [n_head*64]. */
int kh_mla_attend(kh_ctx *ctx, const kh_kv *kv, size_t layer, size_t n_head, const float *q_lat, const float *q_pe,
                  size_t n_positions, float scale, float *out);
/* The same over raw device arrays: c rows 512 wide, pe rows 64 wide. */
int kh_mla_attend_dev(kh_ctx *ctx, size_t n_head, const float *q_lat, const float *q_pe, const float *c,
                      const float *pe, size_t n_positions, float scale, float *out);

/* ---- decode glue (device pointers, asynchronous on the context's stream) */

/* tensor::rms_norm (tensor.rs:329-333) over m rows of n:
 * out = x * (1 / sqrt(mean(x^2) + eps)) * w. */
int kh_rms_norm_dev(kh_ctx *ctx, const float *x, const float *w, size_t m, size_t n, float eps, float *out);
/* Rope::apply (tensor.rs:463-472; interleaved = 0, pairs i and i+half) or
 * Rope::apply_interleaved (tensor.rs:437-446; pairs 2i and 2i+1), in place on
 * x [m][n_vec][2*half], row r at position pos0 + r.  cos_t/sin_t are the
 * caller's tables [max_pos][half] (Rope::tables, tensor.rs:377-387). */
int kh_rope_dev(kh_ctx *ctx, const float *cos_t, const float *sin_t, size_t half, float *x, size_t m,
                size_t n_vec, size_t pos0, int interleaved);
/* swiglu_inplace (tensor.rs:344-350): gate[i] = silu(gate[i]) * up[i]. */
int kh_swiglu_dev(kh_ctx *ctx, float *gate, const float *up, size_t n);
/* softmax_inplace (tensor.rs:297-308) over each of m rows of n, in place. */
int kh_softmax_dev(kh_ctx *ctx, float *x, size_t m, size_t n);

/* ---- mixture of experts ----------------------------------------------- */

/* Router scoring (Scoring, model/ffn.rs:173-177) and selection (Select, ffn.rs:179-195). */
#define KH_SOFTMAX 0
#define KH_SIGMOID 1
#define KH_GREEDY 0
#define KH_GROUP_LIMITED 1
#define KH_NOAUX_TC 2

typedef struct kh_moe kh_moe;

/* Moe (model/ffn.rs:474-506) and its Router (ffn.rs:197-252): n_experts
 * routed experts of width `inter` over `hidden`, top_k picks per token,
 * scoring/select/n_group/topk_group/norm_topk/scale as the router's config,
 * bias (n_experts floats, host) the selection bias of noaux_tc or NULL.
 * The weights are set below as borrowed handles that must outlive the layer. */
int kh_moe_new(kh_ctx *ctx, size_t n_experts, size_t top_k, size_t hidden, size_t inter, int scoring, int select,
               size_t n_group, size_t topk_group, int norm_topk, float scale, const float *bias, kh_moe **out);
int kh_moe_free(kh_moe *moe);
/* The router's gate, [n_experts, hidden], any precision (Moe's gate, ffn.rs:474-506). */
int kh_moe_set_router(kh_moe *moe, const kh_weight *router);
/* Expert `expert`'s Ffn (ffn.rs:355-388): gate/up [inter, hidden], down
 * [hidden, inter]; every expert in one quantised precision. */
int kh_moe_set_expert(kh_moe *moe, size_t expert, const kh_weight *gate, const kh_weight *up, const kh_weight *down);
/* The shared expert (SharedExpert, ffn.rs:413-451; DeepSeek's fused
 * shared experts): gate/up [width, hidden], down [hidden, width]. */
int kh_moe_set_shared(kh_moe *moe, const kh_weight *gate, const kh_weight *up, const kh_weight *down);
/* Moe::run (ffn.rs:615-708): out[m, hidden] for hs[m, hidden].  One token runs
 * as decode_together (ffn.rs:820-842), a batch grouped by expert; both add
 * the experts in expert order after the shared expert, as mix() does. */
int kh_moe_run(kh_ctx *ctx, kh_moe *moe, const float *hs, size_t m, float *out);
int kh_moe_run_dev(kh_ctx *ctx, kh_moe *moe, const float *hs, size_t m, float *out);
/* Router::route (ffn.rs:256-309) for m tokens' logits [m, n_experts]:
 * experts/weights [m, top_k] in pick order (unused slots -1 / 0), count [m]. */
int kh_moe_route(kh_ctx *ctx, const kh_moe *moe, const float *logits, size_t m, int32_t *experts, float *weights,
                 int32_t *count);
/* Parity hook (a debugging aid; no counterpart in the reference): after a
 * kh_moe_run[_dev] of m tokens, the run's intermediates copied to the host,
 * per token and pick, picks in expert order (mix order, ffn.rs:775-805),
 * unused picks zero.  Any pointer may be NULL.  hidden_qs / hidden_scales
 * (the quantised swiglu(gate, up) the down projections read) exist for
 * m > 1 only: one token's stay inside the down GEMV (KH_DECLINED). */
typedef struct kh_moe_picks {
    float *logits;         /* [m][n_experts] router logits */
    int32_t *count;        /* [m] */
    int32_t *experts;      /* [m][top_k] */
    float *weights;        /* [m][top_k] */
    float *gate, *up;      /* [m][top_k][inter] */
    int8_t *hidden_qs;     /* [m][top_k][inter] */
    float *hidden_scales;  /* [m][top_k][inter / 32] */
    float *out;            /* [m][top_k][hidden]: each expert's down projection */
    float *shared_gate, *shared_up;  /* [m][shared width] */
    float *shared_out;     /* [m][hidden] */
} kh_moe_picks;
int kh_debug_moe_picks(kh_ctx *ctx, const kh_moe *moe, size_t m, const kh_moe_picks *out);

/* ---- the quantised-weight cache file ("NANOQ"), read into device weights */

/* The container of crates/llm/src/qcache.rs:30-40 (magic, 64-byte aligned
 * arrays, JSON header at the end, trailing u64 header offset).  The file is
 * mapped and checked as Container::open does (qcache.rs:863-883), every
 * tensor entry parsed as parse_entry does (qcache.rs:817-834) with spans
 * bounds-checked against the file (Container::slice, qcache.rs:906-911).
 * Entries are the CPU engine's q8/q4 (scales + qs spans) and f32 (data), and
 * the GPU backend's GGML q4k, q8 and q4 blocks (crates/gpu/src/qcache.rs:278-296);
 * a kind with no device kernel (q6k) is left out of the table.  Needs no
 * device: provenance checks on the header (Mapped::open, qcache.rs:620-668)
 * are the caller's. */
typedef struct kh_qcache kh_qcache;
int kh_qcache_open(const char *path, kh_qcache **out);
int kh_qcache_free(kh_qcache *qc);
/* The JSON header text (library-owned, valid while the handle lives). */
const char *kh_qcache_header(const kh_qcache *qc);
/* The tensor table in header order. */
int kh_qcache_count(const kh_qcache *qc, size_t *n);
const char *kh_qcache_name(const kh_qcache *qc, size_t i);
/* Precision of the device weight the entry becomes (GGML q8/q4 become KH_Q8/KH_Q4). */
int kh_qcache_info(const kh_qcache *qc, const char *name, int *precision, size_t *rows, size_t *cols);
/* Mapped::vector (qcache.rs:781-790): a [1, n] f32 entry copied to host `out`. */
int kh_qcache_vector(const kh_qcache *qc, const char *name, float *out, size_t n);
/* Mapped::build (qcache.rs:689-713), onto the device: the entry's arrays are
 * copied from the mapping through pinned staging buffers (GGML Q8_0/Q4_0
 * blocks repacked to kvad's q8/q4 layout with f32 scales, exactly). */
int kh_qcache_weight(kh_ctx *ctx, const kh_qcache *qc, const char *name, kh_weight **out);

/* ---- a device-resident decoder (Llama family) ------------------------- */

/* Spec (model/mod.rs:286-330) of a Llama-family decoder: Qwen2/2.5, Llama,
 * Qwen3 dense (llama.rs).  n_ctx bounds the device KV cache. */
typedef struct {
    size_t n_layer, n_embd, n_head, n_kv_head, head_dim, n_ff, vocab, n_ctx;
    float eps;
    int rope_interleaved; /* 0: Rope::apply (HF half split), 1: apply_interleaved */
} kh_llm_spec;

typedef struct kh_llm kh_llm;

/* A session over the model (the Session trait's device-resident backend,
 * model/mod.rs:839-976): weights as borrowed handles, the KV cache in HBM,
 * the greedy next token chosen on the device. */
int kh_llm_new(kh_ctx *ctx, const kh_llm_spec *spec, kh_llm **out);
int kh_llm_free(kh_llm *m);
/* Block l (llama.rs:139-200): q [n_head*hd, n_embd], k/v [n_kv*hd, n_embd],
 * o [n_embd, n_head*hd], gate/up [n_ff, n_embd], down [n_embd, n_ff]; norms
 * and biases are host vectors, copied (biases and q/k norms may be NULL). */
int kh_llm_set_layer(kh_llm *m, size_t l, const kh_weight *q, const kh_weight *k, const kh_weight *v,
                     const kh_weight *o, const kh_weight *gate, const kh_weight *up, const kh_weight *down,
                     const float *attn_norm, const float *mlp_norm, const float *q_b, const float *k_b,
                     const float *v_b, const float *q_norm, const float *k_norm);
/* The ends (llama.rs:384-415): embedding [vocab, n_embd], final norm (host),
 * lm_head or NULL when tied to the embedding. */
int kh_llm_set_ends(kh_llm *m, const kh_weight *embed, const float *final_norm, const kh_weight *lm_head);
/* RoPE tables from Rope::tables (tensor.rs:377-387), host [max_pos, hd/2]. */
int kh_llm_set_rope(kh_llm *m, const float *cos_t, const float *sin_t, size_t max_pos);
/* Session::forward for one token at the next position: logits [vocab] (host,
 * may be NULL) and the greedy next token (sampler::argmax, sampler.rs:217). */
int kh_llm_forward(kh_ctx *ctx, kh_llm *m, int32_t token, float *logits, int32_t *next);
/* Parity hook (a debugging aid; no counterpart in the reference): one
 * kh_llm_forward step of `token` that copies each sub-block's results to the
 * host as it ends.  With L = n_layer, n = the positions held after the step
 * (length before it + 1), qd = n_head * head_dim, kvd = n_kv_head * head_dim:
 * x_embed [n_embd] (the embedding row); per layer qkv [L][qd + 2 kvd] (the
 * projections with biases, before the head norms and RoPE), k_cache / v_cache
 * [L][n][kvd] (the cache after the push), att [L][qd] (attention output),
 * x_attn [L][n_embd] (the residual after the o projection), gate / up
 * [L][n_ff] (quantised weights only), x_mlp [L][n_embd] (the residual after
 * the MLP); logits [vocab].  Any pointer may be NULL. */
typedef struct kh_llm_trace {
    float *x_embed, *qkv, *k_cache, *v_cache, *att, *x_attn, *gate, *up, *x_mlp, *logits;
} kh_llm_trace;
int kh_debug_llm_trace(kh_ctx *ctx, kh_llm *m, int32_t token, const kh_llm_trace *tr);
/* Session::forward(&[u32]) (model/mod.rs:842; CpuSession :1149-1158): n
 * tokens at the next positions of the held sequence, read in passes cut where
 * kh_llm_prefill_pass says.  A pass of m > 1 tokens is the reference's
 * forward_batch (mod.rs:544-549): the embedding rows, run_rows with
 * Rows::Following (llama.rs:224-289: every row rotated and pushed into the
 * held cache, row i attending causally over len + i + 1 positions; the
 * projections on the multi-token GEMV or the int8 GEMM by kh_matmul's rule),
 * and the head over the last row (llama.rs:404-411); a pass of one token is
 * kh_llm_forward's step.  logits [vocab] of the last token (host, may be
 * NULL) and its greedy next token; the cache then holds n more positions.
 * n = 0 does nothing.  Tokens past the vocabulary, or past n_ctx positions,
 * are refused (KH_EINVAL) before anything runs. */
int kh_llm_forward_tokens(kh_ctx *ctx, kh_llm *m, const int32_t *tokens, size_t n, float *logits, int32_t *next);
/* Session::prefill_pass (model/mod.rs:866; CpuSession :1181-1183): how many
 * of `left` prompt tokens the next pass reads -- whole chunks from the front,
 * the rest last.  Feeding kh_llm_forward_tokens a pass at a time, cut here,
 * gives the logits of one call to the bit. */
int kh_llm_prefill_pass(const kh_llm *m, size_t left, size_t *pass);
/* CpuSession::reading (model/mod.rs:1079-1082): `chunk` prompt tokens a pass
 * (at most 65535); 0 restores the default, KVAD_PREFILL_CHUNK
 * (mod.rs:1004-1006) or 64. */
int kh_llm_set_prefill_chunk(kh_llm *m, size_t chunk);
/* Parity hook (no counterpart in the reference): one pass of n tokens as
 * kh_llm_forward_tokens runs it, on the rows path even for n = 1, copying each
 * sub-block's rows out as it ends.  With len = the positions held before the
 * pass: x_embed [n][n_embd]; qkv [L][n][qd + 2 kvd] (before the head norms and
 * RoPE); k_cache / v_cache [L][len + n][kvd]; att [L][n][qd]; x_attn [L][n][n_embd];
 * gate / up [L][n][n_ff] (before swiglu); x_mlp [L][n][n_embd]; logits [vocab]
 * of the last row.  Any pointer may be NULL. */
int kh_debug_llm_trace_pass(kh_ctx *ctx, kh_llm *m, const int32_t *tokens, size_t n, const kh_llm_trace *tr);
/* n greedy steps from `token`, one captured HIP graph replayed per token;
 * tokens[n] receives the tokens generated. */
int kh_llm_generate(kh_ctx *ctx, kh_llm *m, int32_t token, size_t n, int32_t *tokens);
/* n more replays of the captured step from the device state as it stands,
 * asynchronous, nothing copied back (for timing after kh_llm_generate). */
int kh_llm_generate_launch(kh_ctx *ctx, kh_llm *m, size_t n);
/* Session::cached / truncate (model/mod.rs:860-880; KvCache::truncate keeps a prefix). */
int kh_llm_len(const kh_llm *m, size_t *len);
int kh_llm_truncate(kh_llm *m, size_t len);

/* A conversation set aside (the Session trait's Parked, model/mod.rs:837). */
typedef struct kh_llm_parked kh_llm_parked;
/* Session::park (model/mod.rs:883-893, CpuSession :1204-1207): takes the
 * session's cache out, leaving an empty one in its place; pointers move,
 * nothing is copied. */
int kh_llm_park(kh_llm *m, kh_llm_parked **out);
/* Session::resume (model/mod.rs:895-897, :1209-1212): puts a parked cache back
 * in place of the one held, which is dropped.  Consumes `p` (even on error,
 * except KH_EINVAL for a null argument); a cache another session parked is
 * refused ("that cache was not this backend's"). */
int kh_llm_resume(kh_llm *m, kh_llm_parked *p);
/* Drops a parked cache (the Box<dyn Any> going out of scope). */
int kh_llm_parked_free(kh_llm_parked *p);
int kh_llm_parked_len(const kh_llm_parked *p, size_t *len);
/* Session::forward_each (model/mod.rs:899-930, CpuSession :1190-1202;
 * Transformer::forward_each, llama.rs:418-434): tokens[i] onto the end of
 * caches[i], all n in one pass -- one matmul per projection over the n rows,
 * each row attending over its own cache -- and a row of logits for each
 * (logits [n][vocab], host, may be NULL) and its greedy next token (next[n],
 * may be NULL).  The session's own conversation is left as it was.  n == 0
 * does nothing; the caches must be distinct and this session's. */
int kh_llm_forward_each(kh_ctx *ctx, kh_llm *m, size_t n, const int32_t *tokens, kh_llm_parked *const *caches,
                        float *logits, int32_t *next);

#ifdef __cplusplus
}
#endif
#endif
