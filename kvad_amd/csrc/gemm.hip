// Batched prefill: Weight::matmul_bt (crates/llm/src/quant.rs:751-907) and
// tensor::gemm_bt (tensor.rs:102-186).
#include "common.hpp"

namespace kh {

int launch_matmul(kh_ctx *ctx, const kh_weight *w, const float *xs, size_t m, const float *bias, float *y) {
    // Row-at-a-time fallback: one GEMV job per activation row, all in as few
    // launches as the job table allows.  Same per-element arithmetic as the
    // reference's x86 row_dot (quant.rs:865-907).
    const size_t rows = w->rows, cols = w->cols;
    std::vector<GemvJob> jobs(m);
    QAct a{};
    if (w->precision != KH_F32) {
        size_t qb = (m * cols + 255) / 256 * 256, sb = (4 * m * cols / BLOCK + 255) / 256 * 256;
        int rc = ensure(ctx, ctx->ws, qb + 2 * sb);
        if (rc) return rc;
        char *p = static_cast<char *>(ctx->ws.ptr);
        a.qs = reinterpret_cast<int8_t *>(p);
        a.scales = reinterpret_cast<float *>(p + qb);
        a.sums = reinterpret_cast<int32_t *>(p + qb + sb);
        if ((rc = launch_qact(ctx, xs, m, cols, a))) return rc;
    }
    for (size_t i = 0; i < m; i++) {
        GemvJob &j = jobs[i];
        j = GemvJob{};
        j.w = w->qs;
        j.ws = w->scales;
        if (w->precision != KH_F32) {
            j.xq = a.qs + i * cols;
            j.xs = a.scales + i * (cols / BLOCK);
            j.xsum = a.sums + i * (cols / BLOCK);
        } else {
            j.xf = xs + i * cols;
        }
        j.bias = bias;
        j.y = y + i * rows;
        j.rows = (int)rows;
        j.cols = (int)cols;
    }
    return launch_gemv(ctx, w->precision, jobs.data(), (int)m);
}

}  // namespace kh
