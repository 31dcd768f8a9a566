/*
 * kvad_oracle.h -- CPU restatement of kvad's quantised-matmul and
 * decode-attention arithmetic.  TEST INFRASTRUCTURE ONLY: the parity
 * checker for libkvad_hip and the CPU baseline timed beside it.  Nothing in
 * the product links or calls this library.
 *
 * Every function cites the reference (bisand/kvad) lines it restates.  The
 * float arithmetic keeps the reference's operation order and rounding:
 * compiled with -ffp-contract=off because Rust never fuses a*b+c
 * (crates/llm/src/tensor.rs:136-150).
 */
#ifndef KVAD_ORACLE_H
#define KVAD_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVO_BLOCK 32   /* quant.rs:57 */
#define KVO_QK_K 256   /* Q4_K super-block, gpu/src/mpp.rs:241-251 */
#define KVO_Q4K_BYTES 144

/* ---- seeded inputs: nervus xorshift64* + Box-Muller (crates/nervus/src/rng.rs:7-39) ---- */
typedef struct { uint64_t state; } kvo_rng;
void kvo_rng_init(kvo_rng *r, uint64_t seed);
uint64_t kvo_rng_next(kvo_rng *r);
float kvo_rng_uniform(kvo_rng *r);
float kvo_rng_normal(kvo_rng *r);
/* out[i] = rng.normal() * scale, i in order; one generator seeded with `seed`. */
void kvo_fill_normal(uint64_t seed, float scale, float *out, size_t n);

/* ---- threads (model/mod.rs:1096-1123; quant.rs:50-53 one chunk per thread) ---- */
void kvo_set_threads(int n);
int kvo_get_threads(void);

/* ---- quantisation (quant.rs:209-281, 1044-1066) ---- */
void kvo_quantize_q8(const float *w, size_t rows, size_t cols, float *scales, int8_t *qs);
void kvo_quantize_q4(const float *w, size_t rows, size_t cols, float *scales, uint8_t *qs);
/* QActivation::new on one row of n values (n % 32 == 0). */
void kvo_qact(const float *x, size_t n, int8_t *qs, float *scales, int32_t *sums);
/* QActBatch::new: m rows of n values. */
void kvo_qact_batch(const float *xs, size_t m, size_t n, int8_t *qs, float *scales, int32_t *sums);

/* ---- Q4_K codec (build-defined packing of GGML's block_q4_K, mpp.rs:241-315) ---- */
uint16_t kvo_f32_to_f16(float f);
float kvo_f16_to_f32(uint16_t h);
void kvo_q4k_scale_min(const uint8_t *scales12, int j, uint8_t *sc, uint8_t *m);
void kvo_quantize_q4k(const float *w, size_t rows, size_t cols, uint8_t *blocks);

/* ---- dequantised rows: Weight::row (quant.rs:374-402) and the Q4_K decoder (mpp.rs:304-315) ---- */
void kvo_row_q8(const float *scales, const int8_t *qs, size_t cols, size_t r, float *out);
void kvo_row_q4(const float *scales, const uint8_t *qs, size_t cols, size_t r, float *out);
void kvo_row_q4k(const uint8_t *blocks, size_t cols, size_t r, float *out);

/* ---- pass 1 integer block dots (quant.rs:426-440, 168-189) ---- */
/* dots[r * nb + b] for every row r and block b; x quantised by kvo_qact. */
void kvo_block_dots_q8(const int8_t *qs, size_t rows, size_t cols, const int8_t *xq, int32_t *dots);
void kvo_block_dots_q4(const uint8_t *qs, size_t rows, size_t cols, const int8_t *xq,
                       const int32_t *xsums, int32_t *dots);
/* Q4_K: dots[r * nb + b] = sum over the 32 weights of sub-block b of q(0..15) * xq. */
void kvo_block_dots_q4k(const uint8_t *blocks, size_t rows, size_t cols, const int8_t *xq, int32_t *dots);

/* ---- single-token GEMV y = x W^T (+ bias): Weight::matvec_bt (quant.rs:481-512) ---- */
void kvo_matvec_q8(const float *scales, const int8_t *qs, size_t rows, size_t cols,
                   const float *x, const float *bias, float *y);
void kvo_matvec_q4(const float *scales, const uint8_t *qs, size_t rows, size_t cols,
                   const float *x, const float *bias, float *y);
void kvo_matvec_q4k(const uint8_t *blocks, size_t rows, size_t cols, const float *x,
                    const float *bias, float *y);
/* kvo_matvec_q4k organised for the CPU baseline; equal outputs to the bit. */
void kvo_matvec_q4k_fast(const uint8_t *blocks, size_t rows, size_t cols, const float *x, const float *bias,
                         float *y);
/* tensor::matvec_bt (tensor.rs:56-79) */
void kvo_matvec_f32(const float *w, size_t rows, size_t cols, const float *x, const float *bias, float *y);
/* matvec_bt_dequant (quant.rs:522-589), the KVAD_DEQUANT=1 baseline; precision 1=q8, 2=q4 */
void kvo_matvec_dequant(int precision, const float *scales, const void *qs, size_t rows, size_t cols,
                        const float *x, float *y);

/* ---- batched prefill: Weight::matmul_bt x86 path (quant.rs:751-907) ---- */
/* y is [m, rows].  m == 1 goes through matvec, as the reference does. */
void kvo_matmul_q8(const float *scales, const int8_t *qs, size_t rows, size_t cols,
                   const float *xs, size_t m, const float *bias, float *y);
void kvo_matmul_q4(const float *scales, const uint8_t *qs, size_t rows, size_t cols,
                   const float *xs, size_t m, const float *bias, float *y);
void kvo_matmul_q4k(const uint8_t *blocks, size_t rows, size_t cols, const float *xs, size_t m,
                    const float *bias, float *y);
/* tensor::gemm_bt (tensor.rs:102-186): out_t is [rows, m]. */
void kvo_gemm_f32(const float *xs, size_t m, const float *w, size_t rows, size_t cols, float *out_t);
/* Weight::matmul_bt for an f32 weight: gemm_bt then finish (quant.rs:784-787, 849-858). */
void kvo_matmul_f32(const float *w, size_t rows, size_t cols, const float *xs, size_t m,
                    const float *bias, float *y);

/* ---- small f32 pieces (tensor.rs) ---- */
float kvo_dot(const float *a, const float *b, size_t n);            /* tensor.rs:220-235 */
void kvo_softmax(float *x, size_t n);                                 /* tensor.rs:297-308 */
void kvo_rms_norm(const float *x, const float *w, size_t n, float eps, float *out); /* :329-333 */
void kvo_swiglu(float *gate, const float *up, size_t n);              /* tensor.rs:344-350 */
void kvo_rope_tables(size_t head_dim, size_t max_pos, float theta, float *cos_t, float *sin_t); /* :390-407 */
void kvo_rope_apply(const float *cos_t, const float *sin_t, size_t half, float *x, size_t pos); /* :463-472 */
void kvo_rope_apply_interleaved(const float *cos_t, const float *sin_t, size_t half, float *x, size_t pos); /* :437-446 */

/* ---- decode attention: model::attend (model/mod.rs:769-819) ---- */
/* k_cache/v_cache rows are n_kv_head*head_dim wide; out is n_head*head_dim. */
void kvo_attend(size_t n_head, size_t n_kv_head, size_t head_dim, const float *q,
                const float *k_cache, const float *v_cache, size_t n_positions, float *out);

/* ---- latent attention, absorbed: model/deepseek.rs:553-591 ---- */
/* c_cache rows are lat wide, pe_cache rows rope wide; out is n_head*lat (the
 * attended latent of each head, before uv). */
void kvo_mla_attend(size_t n_head, size_t lat, size_t rope, const float *q_lat, const float *q_pe,
                    const float *c_cache, const float *pe_cache, size_t n_positions, float scale, float *out);

/* ---- MoE router: Router::route (model/ffn.rs:256-309) ---- */
/* scoring 0 = softmax, 1 = sigmoid; select 0 greedy, 1 group-limited, 2 noaux_tc.
 * Writes up to top_k (expert, weight) pairs in pick order; returns how many. */
int kvo_route(const float *logits, size_t n_experts, size_t top_k, int scoring, int select,
              size_t n_group, size_t topk_group, int norm_topk, float scale, const float *bias,
              int32_t *experts, float *weights);

/* ---- MoE layer: Moe::run (model/ffn.rs:615-708), every weight q8 ---- */
/* Expert x's gate/up occupy rows [x*inter, (x+1)*inter) of g/u ([n_exp*inter, hidden]),
 * its down rows [x*hidden, (x+1)*hidden) of d ([n_exp*hidden, inter]); scales alike.
 * sh_inter == 0 means no shared expert.  out is [m, hidden]. */
void kvo_moe_run_q8(const float *hs, size_t m, size_t hidden, size_t inter, size_t n_exp, size_t top_k,
                    int scoring, int select, size_t n_group, size_t topk_group, int norm_topk, float scale,
                    const float *bias, const float *r_s, const int8_t *r_q, const float *g_s, const int8_t *g_q,
                    const float *u_s, const int8_t *u_q, const float *d_s, const int8_t *d_q, size_t sh_inter,
                    const float *sg_s, const int8_t *sg_q, const float *su_s, const int8_t *su_q,
                    const float *sd_s, const int8_t *sd_q, float *out);

#ifdef __cplusplus
}
#endif
#endif
