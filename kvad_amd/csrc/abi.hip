// The C ABI of libkvad_hip (include/kvad_hip.h): contexts, weight upload,
// the KV cache, and the entry points that stage host buffers around the
// kernel launchers.
#include <cstring>
#include <memory>

#include "common.hpp"

namespace kh {

static thread_local std::string g_error;

void set_error(const std::string &msg) { g_error = msg; }

int fail(int code, const std::string &msg) {
    set_error(msg);
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? KH_ENOMEM : KH_EHIP;
}

int ensure(kh_ctx *ctx, Workspace &w, size_t bytes) {
    if (bytes <= w.bytes) return KH_OK;
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    want = (want + 4095) / 4096 * 4096;
    if (w.ptr) {
        KH_HIP(hipStreamSynchronize(ctx->stream));
        KH_HIP(hipFree(w.ptr));
        w.ptr = nullptr;
        w.bytes = 0;
    }
    KH_HIP(hipMalloc(&w.ptr, want));
    w.bytes = want;
    return KH_OK;
}

namespace {

constexpr size_t ALIGN = 256;
inline size_t up(size_t n) { return (n + ALIGN - 1) / ALIGN * ALIGN; }

struct Guard {
    std::lock_guard<std::recursive_mutex> lock;
    explicit Guard(kh_ctx *c) : lock(c->mu) { (void)hipSetDevice(c->device); }
};

int check_weight(const kh_weight *w) {
    if (!w || !w->ctx) return fail(KH_EINVAL, "null weight");
    return KH_OK;
}

// Carves the quantised activation for m rows of k values out of `base`.
QAct carve_qact(char *base, size_t m, size_t k, size_t *used) {
    QAct a;
    size_t off = 0;
    a.qs = reinterpret_cast<int8_t *>(base + off);
    off += up(m * k);
    a.scales = reinterpret_cast<float *>(base + off);
    off += up(4 * m * k / BLOCK);
    a.sums = reinterpret_cast<int32_t *>(base + off);
    off += up(4 * m * k / BLOCK);
    *used = off;
    return a;
}

size_t qact_bytes(size_t m, size_t k) { return up(m * k) + 2 * up(4 * m * k / BLOCK); }

GemvJob job_for(const kh_weight *w, const QAct *a, const float *xf, const float *bias, float *y, int32_t *dots) {
    GemvJob j{};
    j.w = w->qs;
    j.ws = w->scales;
    if (a) {
        j.xq = a->qs;
        j.xs = a->scales;
        j.xsum = a->sums;
    }
    j.xf = xf;
    j.bias = bias;
    j.y = y;
    j.dots = dots;
    j.rows = (int)w->rows;
    j.cols = (int)w->cols;
    return j;
}

// The GEMV jobs for n matvecs on device pointers, quantising into ws the
// inputs of wide rows (once per distinct input, quant.rs:634-644).
int make_jobs(kh_ctx *ctx, size_t n, const kh_weight *const *w, const float *const *x, const float *const *bias,
              float *const *y, int32_t *dots, std::vector<GemvJob> &jobs) {
    size_t total = 0;
    for (size_t i = 0; i < n; i++)
        if (w[i]->precision != KH_F32 && w[i]->cols > fuse_max_cols(w[i]->precision)) total += qact_bytes(1, w[i]->cols);
    int rc = total ? ensure(ctx, ctx->ws, total) : KH_OK;
    if (rc) return rc;
    char *p = static_cast<char *>(ctx->ws.ptr);
    QAct last{};
    jobs.clear();
    for (size_t i = 0; i < n; i++) {
        const float *b = bias ? bias[i] : nullptr;
        if (w[i]->precision == KH_F32 || w[i]->cols <= fuse_max_cols(w[i]->precision)) {
            jobs.push_back(job_for(w[i], nullptr, x[i], b, y[i], dots));
            continue;
        }
        if (!(i > 0 && x[i] == x[i - 1] && w[i]->cols == w[i - 1]->cols && last.qs)) {
            size_t used;
            last = carve_qact(p, 1, w[i]->cols, &used);
            p += used;
            if ((rc = launch_qact(ctx, x[i], 1, w[i]->cols, last))) return rc;
        }
        jobs.push_back(job_for(w[i], &last, nullptr, b, y[i], dots));
    }
    return KH_OK;
}

}  // namespace

// matvec on device pointers.
int matvec_device(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y, int32_t *dots) {
    // KVAD_DEQUANT=1 selects the dequantising kernel (quant.rs:485-486); the
    // block-dot hook always reads the integer path
    if (!dots && w->precision != KH_F32 && dequant_selected()) return launch_gemv_dequant(ctx, w, x, bias, y);
    std::vector<GemvJob> jobs;
    int rc = make_jobs(ctx, 1, &w, &x, &bias, &y, dots, jobs);
    if (rc) return rc;
    return launch_gemv(ctx, w->precision, jobs.data(), 1);
}

int matvec_many_device(kh_ctx *ctx, size_t n, const kh_weight *const *w, const float *const *x,
                       float *const *y) {
    if (n == 0) return KH_OK;
    for (size_t i = 0; i < n; i++) {
        if (check_weight(w[i])) return KH_EINVAL;
        if (w[i]->precision == KH_F32) return fail(KH_DECLINED, "matvec_many: an f32 weight is not this call's to run");
    }
    // quant.rs:629-633: None when the dequantising kernel was asked for
    if (dequant_selected()) return fail(KH_DECLINED, "matvec_many: KVAD_DEQUANT asks for one matvec at a time");
    std::vector<GemvJob> all;
    int rc = make_jobs(ctx, n, w, x, nullptr, y, nullptr, all);
    if (rc) return rc;
    // One launch per precision present; a single precision is one launch.
    for (int prec : {KH_Q8, KH_Q4, KH_Q4K}) {
        std::vector<GemvJob> jobs;
        for (size_t i = 0; i < n; i++)
            if (w[i]->precision == prec) jobs.push_back(all[i]);
        if (!jobs.empty() && (rc = launch_gemv(ctx, prec, jobs.data(), (int)jobs.size()))) return rc;
    }
    return KH_OK;
}

int matmul_device(kh_ctx *ctx, const kh_weight *w, const float *xs, size_t m, const float *bias, float *y) {
    if (m == 1) return matvec_device(ctx, w, xs, bias, y, nullptr);
    return launch_matmul(ctx, w, xs, m, bias, y);
}

namespace {
}  // namespace
}  // namespace kh

using namespace kh;

extern "C" {

const char *kh_last_error(void) { return g_error.c_str(); }

const char *kh_version(void) { return "kvad_hip 0.1.0 (gfx950)"; }

int kh_init(int device, kh_ctx **out) {
    if (!out) return fail(KH_EINVAL, "kh_init: out is null");
    *out = nullptr;
    int n = 0;
    KH_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(KH_EINVAL, "kh_init: no such device");
    KH_HIP(hipSetDevice(device));
    std::unique_ptr<kh_ctx> ctx(new kh_ctx());
    ctx->device = device;
    KH_HIP(hipDeviceGetAttribute(&ctx->cu_count, hipDeviceAttributeMultiprocessorCount, device));
    KH_HIP(hipStreamCreateWithFlags(&ctx->own, hipStreamNonBlocking));
    ctx->stream = ctx->own;
    // once per device: the no-allocation entry points' array.  Not fatal:
    // without it only kh_attend_dev_noalloc refuses (KH_EINVAL).
    (void)scratch_init(device);
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipStreamDestroy(ctx->own);
        return hip_fail(e, "hipDeviceSynchronize");
    }
    *out = ctx.release();
    return KH_OK;
}

int kh_free(kh_ctx *ctx) {
    if (!ctx) return KH_OK;
    {
        Guard g(ctx);
        (void)hipStreamSynchronize(ctx->stream);
        if (ctx->ws.ptr) (void)hipFree(ctx->ws.ptr);
        if (ctx->io.ptr) (void)hipFree(ctx->io.ptr);
        if (ctx->moe.ptr) (void)hipFree(ctx->moe.ptr);
        if (ctx->gemm.ptr) (void)hipFree(ctx->gemm.ptr);
        if (ctx->own) (void)hipStreamDestroy(ctx->own);
    }
    delete ctx;
    return KH_OK;
}

int kh_set_stream(kh_ctx *ctx, void *stream) {
    if (!ctx) return fail(KH_EINVAL, "null context");
    Guard g(ctx);
    KH_HIP(hipStreamSynchronize(ctx->stream));
    ctx->stream = stream ? static_cast<hipStream_t>(stream) : ctx->own;
    return KH_OK;
}

int kh_synchronize(kh_ctx *ctx) {
    if (!ctx) return fail(KH_EINVAL, "null context");
    Guard g(ctx);
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

int kh_reserve(kh_ctx *ctx, size_t bytes) {
    if (!ctx) return fail(KH_EINVAL, "null context");
    Guard g(ctx);
    return ensure(ctx, ctx->ws, bytes);
}

// ---- weights -------------------------------------------------------------

static int upload(kh_ctx *ctx, int precision, size_t rows, size_t cols, const void *qs, size_t qs_bytes,
                  const float *scales, size_t n_scales, kh_weight **out) {
    std::unique_ptr<kh_weight> w(new kh_weight());
    w->ctx = ctx;
    w->precision = precision;
    w->rows = rows;
    w->cols = cols;
    KH_HIP(hipMalloc(&w->qs, qs_bytes ? qs_bytes : 16));
    KH_HIP(hipMemcpy(w->qs, qs, qs_bytes, hipMemcpyHostToDevice));
    w->bytes = qs_bytes;
    if (n_scales) {
        KH_HIP(hipMalloc(reinterpret_cast<void **>(&w->scales), 4 * n_scales));
        KH_HIP(hipMemcpy(w->scales, scales, 4 * n_scales, hipMemcpyHostToDevice));
        w->bytes += 4 * n_scales;
    }
    *out = w.release();
    return KH_OK;
}

static int shape_check(size_t rows, size_t cols, size_t multiple, const char *what) {
    if (rows == 0 || cols == 0 || cols % multiple != 0 || rows > (size_t)INT32_MAX || cols > (size_t)INT32_MAX)
        return fail(KH_EINVAL, std::string(what) + ": needs rows > 0 and cols a positive multiple of " +
                                   std::to_string(multiple));
    return KH_OK;
}

int kh_weight_q8(kh_ctx *ctx, size_t rows, size_t cols, const float *scales, const int8_t *qs, kh_weight **out) {
    if (!ctx || !out || !scales || !qs) return fail(KH_EINVAL, "kh_weight_q8: null argument");
    if (shape_check(rows, cols, BLOCK, "kh_weight_q8")) return KH_EINVAL;
    Guard g(ctx);
    return upload(ctx, KH_Q8, rows, cols, qs, rows * cols, scales, rows * cols / BLOCK, out);
}

int kh_weight_q4(kh_ctx *ctx, size_t rows, size_t cols, const float *scales, const uint8_t *qs, kh_weight **out) {
    if (!ctx || !out || !scales || !qs) return fail(KH_EINVAL, "kh_weight_q4: null argument");
    if (shape_check(rows, cols, BLOCK, "kh_weight_q4")) return KH_EINVAL;
    Guard g(ctx);
    return upload(ctx, KH_Q4, rows, cols, qs, rows * cols / 2, scales, rows * cols / BLOCK, out);
}

int kh_weight_q4k(kh_ctx *ctx, size_t rows, size_t cols, const uint8_t *blocks, kh_weight **out) {
    if (!ctx || !out || !blocks) return fail(KH_EINVAL, "kh_weight_q4k: null argument");
    if (shape_check(rows, cols, QK_K, "kh_weight_q4k")) return KH_EINVAL;
    Guard g(ctx);
    return upload(ctx, KH_Q4K, rows, cols, blocks, rows * (cols / QK_K) * Q4K_BYTES, nullptr, 0, out);
}

int kh_weight_f32(kh_ctx *ctx, size_t rows, size_t cols, const float *data, kh_weight **out) {
    if (!ctx || !out || !data) return fail(KH_EINVAL, "kh_weight_f32: null argument");
    if (shape_check(rows, cols, 1, "kh_weight_f32")) return KH_EINVAL;
    Guard g(ctx);
    return upload(ctx, KH_F32, rows, cols, data, 4 * rows * cols, nullptr, 0, out);
}

static size_t qs_bytes_of(int precision, size_t rows, size_t cols) {
    switch (precision) {
        case KH_Q8: return rows * cols;
        case KH_Q4: return rows * cols / 2;
        case KH_Q4K: return rows * (cols / QK_K) * Q4K_BYTES;
        default: return 4 * rows * cols;
    }
}

static int quantize(kh_ctx *ctx, size_t rows, size_t cols, const float *data, int precision, bool host,
                    kh_weight **out) {
    if (!ctx || !out || !data) return fail(KH_EINVAL, "kh_weight_quantize: null argument");
    if (precision != KH_F32 && precision != KH_Q8 && precision != KH_Q4 && precision != KH_Q4K)
        return fail(KH_EINVAL, "kh_weight_quantize: unknown precision");
    if (shape_check(rows, cols, 1, "kh_weight_quantize")) return KH_EINVAL;
    // A width that does not block stays f32, as Weight::quantize keeps it
    // (quant.rs:211-213).
    const size_t unit = precision == KH_Q4K ? QK_K : BLOCK;
    if (cols % unit != 0 || cols < unit) precision = KH_F32;
    Guard g(ctx);
    if (precision == KH_F32) {
        std::unique_ptr<kh_weight> w(new kh_weight());
        w->ctx = ctx;
        w->precision = KH_F32;
        w->rows = rows;
        w->cols = cols;
        w->bytes = 4 * rows * cols;
        KH_HIP(hipMalloc(&w->qs, w->bytes));
        hipError_t e = hipMemcpyAsync(w->qs, data, w->bytes, host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice,
                                      ctx->stream);
        if (e == hipSuccess && host) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            (void)hipFree(w->qs);
            return hip_fail(e, "kh_weight_quantize: copy");
        }
        *out = w.release();
        return KH_OK;
    }
    std::unique_ptr<kh_weight> w(new kh_weight());
    w->ctx = ctx;
    w->precision = precision;
    w->rows = rows;
    w->cols = cols;
    size_t qb = qs_bytes_of(precision, rows, cols);
    KH_HIP(hipMalloc(&w->qs, qb));
    w->bytes = qb;
    if (precision != KH_Q4K) {
        KH_HIP(hipMalloc(reinterpret_cast<void **>(&w->scales), 4 * rows * cols / BLOCK));
        w->bytes += 4 * rows * cols / BLOCK;
    }
    const float *src = data;
    float *tmp = nullptr;
    if (host) {
        KH_HIP(hipMalloc(reinterpret_cast<void **>(&tmp), 4 * rows * cols));
        KH_HIP(hipMemcpyAsync(tmp, data, 4 * rows * cols, hipMemcpyHostToDevice, ctx->stream));
        src = tmp;
    }
    int rc = launch_quantize(ctx, src, rows, cols, precision, w->qs, w->scales);
    if (host) {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        (void)hipFree(tmp);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    }
    if (rc) {
        (void)hipFree(w->qs);
        if (w->scales) (void)hipFree(w->scales);
        return rc;
    }
    *out = w.release();
    return KH_OK;
}

int kh_weight_quantize(kh_ctx *ctx, size_t rows, size_t cols, const float *data, int precision, kh_weight **out) {
    return quantize(ctx, rows, cols, data, precision, true, out);
}

int kh_weight_quantize_dev(kh_ctx *ctx, size_t rows, size_t cols, const float *data, int precision,
                           kh_weight **out) {
    return quantize(ctx, rows, cols, data, precision, false, out);
}

int kh_weight_parts(const kh_weight *w, void *qs, float *scales) {
    if (check_weight(w) || !qs) return fail(KH_EINVAL, "kh_weight_parts: null argument");
    Guard g(w->ctx);
    KH_HIP(hipMemcpyAsync(qs, w->qs, qs_bytes_of(w->precision, w->rows, w->cols), hipMemcpyDeviceToHost,
                          w->ctx->stream));
    if (w->scales && scales)
        KH_HIP(hipMemcpyAsync(scales, w->scales, 4 * w->rows * w->cols / BLOCK, hipMemcpyDeviceToHost, w->ctx->stream));
    KH_HIP(hipStreamSynchronize(w->ctx->stream));
    return KH_OK;
}

int kh_weight_free(kh_weight *w) {
    if (!w) return KH_OK;
    if (w->ctx) {
        Guard g(w->ctx);
        (void)hipStreamSynchronize(w->ctx->stream);
        if (w->qs) (void)hipFree(w->qs);
        if (w->scales) (void)hipFree(w->scales);
    }
    delete w;
    return KH_OK;
}

int kh_weight_info(const kh_weight *w, size_t *rows, size_t *cols, int *precision, size_t *bytes) {
    if (check_weight(w)) return KH_EINVAL;
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    if (precision) *precision = w->precision;
    if (bytes) *bytes = w->bytes;
    return KH_OK;
}

int kh_weight_row(kh_ctx *ctx, const kh_weight *w, size_t r, float *out) {
    if (!ctx || check_weight(w) || !out) return fail(KH_EINVAL, "kh_weight_row: null argument");
    if (r >= w->rows) return fail(KH_EINVAL, "kh_weight_row: row out of range");
    Guard g(ctx);
    int rc = ensure(ctx, ctx->io, 4 * w->cols);
    if (rc) return rc;
    float *d = static_cast<float *>(ctx->io.ptr);
    if ((rc = launch_dequant_row(ctx, w, r, d))) return rc;
    KH_HIP(hipMemcpyAsync(out, d, 4 * w->cols, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

// ---- GEMV / GEMM -----------------------------------------------------------

int kh_matvec_dev(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y) {
    if (!ctx || check_weight(w) || !x || !y) return fail(KH_EINVAL, "kh_matvec_dev: null argument");
    Guard g(ctx);
    return matvec_device(ctx, w, x, bias, y, nullptr);
}

static int matvec_host(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y,
                       int32_t *dots) {
    Guard g(ctx);
    const size_t rows = w->rows, cols = w->cols, nb = cols / BLOCK;
    size_t bytes = up(4 * cols) + 2 * up(4 * rows) + (dots ? up(4 * rows * nb) : 0);
    int rc = ensure(ctx, ctx->io, bytes);
    if (rc) return rc;
    char *p = static_cast<char *>(ctx->io.ptr);
    float *dx = reinterpret_cast<float *>(p);
    float *dy = reinterpret_cast<float *>(p + up(4 * cols));
    float *db = reinterpret_cast<float *>(p + up(4 * cols) + up(4 * rows));
    int32_t *dd = dots ? reinterpret_cast<int32_t *>(p + up(4 * cols) + 2 * up(4 * rows)) : nullptr;
    KH_HIP(hipMemcpyAsync(dx, x, 4 * cols, hipMemcpyHostToDevice, ctx->stream));
    if (bias) KH_HIP(hipMemcpyAsync(db, bias, 4 * rows, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = matvec_device(ctx, w, dx, bias ? db : nullptr, dy, dd))) return rc;
    KH_HIP(hipMemcpyAsync(y, dy, 4 * rows, hipMemcpyDeviceToHost, ctx->stream));
    if (dots) KH_HIP(hipMemcpyAsync(dots, dd, 4 * rows * nb, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

int kh_matvec(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y) {
    if (!ctx || check_weight(w) || !x || !y) return fail(KH_EINVAL, "kh_matvec: null argument");
    return matvec_host(ctx, w, x, bias, y, nullptr);
}

int kh_matvec_dequant_dev(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y) {
    if (!ctx || check_weight(w) || !x || !y) return fail(KH_EINVAL, "kh_matvec_dequant_dev: null argument");
    Guard g(ctx);
    return launch_gemv_dequant(ctx, w, x, bias, y);
}

int kh_matvec_dequant(kh_ctx *ctx, const kh_weight *w, const float *x, const float *bias, float *y) {
    if (!ctx || check_weight(w) || !x || !y) return fail(KH_EINVAL, "kh_matvec_dequant: null argument");
    if (w->precision == KH_F32) return fail(KH_EINVAL, "kh_matvec_dequant: f32 weights have nothing to dequantise");
    Guard g(ctx);
    const size_t rows = w->rows, cols = w->cols;
    int rc = ensure(ctx, ctx->io, up(4 * cols) + 2 * up(4 * rows));
    if (rc) return rc;
    char *p = static_cast<char *>(ctx->io.ptr);
    float *dx = reinterpret_cast<float *>(p);
    float *dy = reinterpret_cast<float *>(p + up(4 * cols));
    float *db = reinterpret_cast<float *>(p + up(4 * cols) + up(4 * rows));
    KH_HIP(hipMemcpyAsync(dx, x, 4 * cols, hipMemcpyHostToDevice, ctx->stream));
    if (bias) KH_HIP(hipMemcpyAsync(db, bias, 4 * rows, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = launch_gemv_dequant(ctx, w, dx, bias ? db : nullptr, dy))) return rc;
    KH_HIP(hipMemcpyAsync(y, dy, 4 * rows, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

int kh_debug_block_dots(kh_ctx *ctx, const kh_weight *w, const float *x, int32_t *dots) {
    if (!ctx || check_weight(w) || !x || !dots) return fail(KH_EINVAL, "kh_debug_block_dots: null argument");
    if (w->precision == KH_F32) return fail(KH_EINVAL, "kh_debug_block_dots: f32 weights have no block dots");
    std::vector<float> y(w->rows);
    return matvec_host(ctx, w, x, nullptr, y.data(), dots);
}

int kh_debug_stream_dev(kh_ctx *ctx, size_t n, const kh_weight *const *w, uint32_t *sink) {
    if (!ctx || !sink || (n && !w)) return fail(KH_EINVAL, "kh_debug_stream_dev: null argument");
    if (n > 4) return fail(KH_EINVAL, "kh_debug_stream_dev: at most four weights a launch");
    for (size_t i = 0; i < n; i++)
        if (check_weight(w[i])) return KH_EINVAL;
    Guard g(ctx);
    return launch_stream(ctx, n, w, sink);
}

int kh_debug_qact(kh_ctx *ctx, const float *x, size_t n, int8_t *qs, float *scales, int32_t *sums) {
    if (!ctx || !x || !qs || !scales || !sums) return fail(KH_EINVAL, "kh_debug_qact: null argument");
    if (n % BLOCK) return fail(KH_EINVAL, "kh_debug_qact: n must be a multiple of 32");
    Guard g(ctx);
    int rc = ensure(ctx, ctx->io, up(4 * n) + qact_bytes(1, n));
    if (rc) return rc;
    char *p = static_cast<char *>(ctx->io.ptr);
    float *dx = reinterpret_cast<float *>(p);
    size_t used;
    QAct a = carve_qact(p + up(4 * n), 1, n, &used);
    KH_HIP(hipMemcpyAsync(dx, x, 4 * n, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = launch_qact(ctx, dx, 1, n, a))) return rc;
    KH_HIP(hipMemcpyAsync(qs, a.qs, n, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipMemcpyAsync(scales, a.scales, 4 * (n / BLOCK), hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipMemcpyAsync(sums, a.sums, 4 * (n / BLOCK), hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

int kh_debug_quant_check(kh_ctx *ctx, uint64_t *counts) {
    if (!ctx || !counts) return fail(KH_EINVAL, "kh_debug_quant_check: null argument");
    Guard g(ctx);
    int rc = ensure(ctx, ctx->io, 256);
    if (rc) return rc;
    unsigned long long *d = static_cast<unsigned long long *>(ctx->io.ptr);
    KH_HIP(hipMemsetAsync(d, 0, 3 * sizeof(unsigned long long), ctx->stream));
    if ((rc = launch_quant_check(ctx, d))) return rc;
    KH_HIP(hipMemcpyAsync(counts, d, 3 * sizeof(unsigned long long), hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

int kh_qact_dev(kh_ctx *ctx, const float *x, size_t m, size_t n, int8_t *qs, float *scales, int32_t *sums) {
    if (!ctx || !x || !qs || !scales || !sums) return fail(KH_EINVAL, "kh_qact_dev: null argument");
    if (n % BLOCK) return fail(KH_EINVAL, "kh_qact_dev: n must be a multiple of 32");
    Guard g(ctx);
    QAct a{qs, scales, sums};
    return launch_qact(ctx, x, m, n, a);
}

int kh_matvec_q_dev(kh_ctx *ctx, const kh_weight *w, const int8_t *qs, const float *scales, const int32_t *sums,
                    const float *bias, float *y) {
    if (!ctx || check_weight(w) || !qs || !scales || !sums || !y) return fail(KH_EINVAL, "kh_matvec_q_dev: null argument");
    if (w->precision == KH_F32) return fail(KH_EINVAL, "kh_matvec_q_dev: f32 weights take kh_matvec_dev");
    Guard g(ctx);
    QAct a{const_cast<int8_t *>(qs), const_cast<float *>(scales), const_cast<int32_t *>(sums)};
    GemvJob j = job_for(w, &a, nullptr, bias, y, nullptr);
    return launch_gemv(ctx, w->precision, &j, 1);
}

int kh_matvec_many_dev(kh_ctx *ctx, size_t n, const kh_weight *const *w, const float *const *x, float *const *y) {
    if (!ctx || (n && (!w || !x || !y))) return fail(KH_EINVAL, "kh_matvec_many_dev: null argument");
    Guard g(ctx);
    return matvec_many_device(ctx, n, w, x, y);
}

int kh_matvec_many(kh_ctx *ctx, size_t n, const kh_weight *const *w, const float *const *x, float *const *y) {
    if (!ctx || (n && (!w || !x || !y))) return fail(KH_EINVAL, "kh_matvec_many: null argument");
    Guard g(ctx);
    for (size_t i = 0; i < n; i++) {
        if (check_weight(w[i])) return KH_EINVAL;
        if (w[i]->precision == KH_F32) return fail(KH_DECLINED, "matvec_many: an f32 weight is not this call's to run");
    }
    size_t bytes = 0;
    for (size_t i = 0; i < n; i++) bytes += up(4 * w[i]->cols) + up(4 * w[i]->rows);
    int rc = ensure(ctx, ctx->io, bytes);
    if (rc) return rc;
    char *p = static_cast<char *>(ctx->io.ptr);
    std::vector<const float *> dx(n);
    std::vector<float *> dy(n);
    for (size_t i = 0; i < n; i++) {
        // the same host input twice in a row stays one device input, so that
        // the adjacent-job dedupe sees it too
        if (i > 0 && x[i] == x[i - 1] && w[i]->cols == w[i - 1]->cols) {
            dx[i] = dx[i - 1];
        } else {
            float *d = reinterpret_cast<float *>(p);
            p += up(4 * w[i]->cols);
            KH_HIP(hipMemcpyAsync(d, x[i], 4 * w[i]->cols, hipMemcpyHostToDevice, ctx->stream));
            dx[i] = d;
        }
        dy[i] = reinterpret_cast<float *>(p);
        p += up(4 * w[i]->rows);
    }
    if ((rc = matvec_many_device(ctx, n, w, dx.data(), dy.data()))) return rc;
    for (size_t i = 0; i < n; i++)
        KH_HIP(hipMemcpyAsync(y[i], dy[i], 4 * w[i]->rows, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

int kh_matmul_dev(kh_ctx *ctx, const kh_weight *w, const float *xs, size_t m, const float *bias, float *y) {
    if (!ctx || check_weight(w) || !xs || !y) return fail(KH_EINVAL, "kh_matmul_dev: null argument");
    if (m == 0) return KH_OK;
    Guard g(ctx);
    return matmul_device(ctx, w, xs, m, bias, y);
}

int kh_matmul(kh_ctx *ctx, const kh_weight *w, const float *xs, size_t m, const float *bias, float *y) {
    if (!ctx || check_weight(w) || !xs || !y) return fail(KH_EINVAL, "kh_matmul: null argument");
    if (m == 0) return KH_OK;
    Guard g(ctx);
    const size_t rows = w->rows, cols = w->cols;
    size_t bytes = up(4 * m * cols) + up(4 * m * rows) + up(4 * rows);
    int rc = ensure(ctx, ctx->io, bytes);
    if (rc) return rc;
    char *p = static_cast<char *>(ctx->io.ptr);
    float *dx = reinterpret_cast<float *>(p);
    float *dy = reinterpret_cast<float *>(p + up(4 * m * cols));
    float *db = reinterpret_cast<float *>(p + up(4 * m * cols) + up(4 * m * rows));
    KH_HIP(hipMemcpyAsync(dx, xs, 4 * m * cols, hipMemcpyHostToDevice, ctx->stream));
    if (bias) KH_HIP(hipMemcpyAsync(db, bias, 4 * rows, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = matmul_device(ctx, w, dx, m, bias ? db : nullptr, dy))) return rc;
    KH_HIP(hipMemcpyAsync(y, dy, 4 * m * rows, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

// ---- KV cache --------------------------------------------------------------

int kh_kv_new(kh_ctx *ctx, size_t n_layer, size_t k_dim, size_t v_dim, size_t capacity, kh_kv **out) {
    if (!ctx || !out) return fail(KH_EINVAL, "kh_kv_new: null argument");
    if (n_layer == 0 || k_dim == 0 || v_dim == 0 || k_dim % 4 || v_dim % 4)
        return fail(KH_EINVAL, "kh_kv_new: needs layers and widths that are positive multiples of 4");
    Guard g(ctx);
    std::unique_ptr<kh_kv> kv(new kh_kv());
    kv->ctx = ctx;
    kv->n_layer = n_layer;
    kv->k_dim = k_dim;
    kv->v_dim = v_dim;
    kv->capacity = capacity ? capacity : 256;  // FIRST, gpu/src/common.rs:547-700
    kv->k.assign(n_layer, nullptr);
    kv->v.assign(n_layer, nullptr);
    kv->rows.assign(n_layer, 0);
    for (size_t l = 0; l < n_layer; l++) {
        KH_HIP(hipMalloc(reinterpret_cast<void **>(&kv->k[l]), 4 * kv->capacity * k_dim));
        KH_HIP(hipMalloc(reinterpret_cast<void **>(&kv->v[l]), 4 * kv->capacity * v_dim));
    }
    *out = kv.release();
    return KH_OK;
}

int kh_kv_free(kh_kv *kv) {
    if (!kv) return KH_OK;
    {
        Guard g(kv->ctx);
        (void)hipStreamSynchronize(kv->ctx->stream);
        for (size_t l = 0; l < kv->n_layer; l++) {
            if (kv->k[l]) (void)hipFree(kv->k[l]);
            if (kv->v[l]) (void)hipFree(kv->v[l]);
        }
    }
    delete kv;
    return KH_OK;
}

// Doubles every layer's arrays until `need` positions fit.
static int kv_grow(kh_kv *kv, size_t need) {
    if (need <= kv->capacity) return KH_OK;
    size_t cap = kv->capacity;
    while (cap < need) cap *= 2;
    kh_ctx *ctx = kv->ctx;
    for (size_t l = 0; l < kv->n_layer; l++) {
        float *nk = nullptr, *nv = nullptr;
        KH_HIP(hipMalloc(reinterpret_cast<void **>(&nk), 4 * cap * kv->k_dim));
        KH_HIP(hipMalloc(reinterpret_cast<void **>(&nv), 4 * cap * kv->v_dim));
        KH_HIP(hipMemcpyAsync(nk, kv->k[l], 4 * kv->rows[l] * kv->k_dim, hipMemcpyDeviceToDevice, ctx->stream));
        KH_HIP(hipMemcpyAsync(nv, kv->v[l], 4 * kv->rows[l] * kv->v_dim, hipMemcpyDeviceToDevice, ctx->stream));
        KH_HIP(hipStreamSynchronize(ctx->stream));
        KH_HIP(hipFree(kv->k[l]));
        KH_HIP(hipFree(kv->v[l]));
        kv->k[l] = nk;
        kv->v[l] = nv;
    }
    kv->capacity = cap;
    return KH_OK;
}

static int kv_push(kh_kv *kv, size_t layer, const float *k, const float *v, size_t m, hipMemcpyKind kind) {
    if (!kv || !k || !v) return fail(KH_EINVAL, "kh_kv_push: null argument");
    if (layer >= kv->n_layer) return fail(KH_EINVAL, "kh_kv_push: no such layer");
    if (m == 0) return KH_OK;
    Guard g(kv->ctx);
    int rc = kv_grow(kv, kv->rows[layer] + m);
    if (rc) return rc;
    size_t r = kv->rows[layer];
    KH_HIP(hipMemcpyAsync(kv->k[layer] + r * kv->k_dim, k, 4 * m * kv->k_dim, kind, kv->ctx->stream));
    KH_HIP(hipMemcpyAsync(kv->v[layer] + r * kv->v_dim, v, 4 * m * kv->v_dim, kind, kv->ctx->stream));
    if (kind == hipMemcpyHostToDevice) KH_HIP(hipStreamSynchronize(kv->ctx->stream));
    kv->rows[layer] = r + m;
    return KH_OK;
}

int kh_kv_push(kh_kv *kv, size_t layer, const float *k, const float *v, size_t m) {
    return kv_push(kv, layer, k, v, m, hipMemcpyHostToDevice);
}

int kh_kv_push_dev(kh_kv *kv, size_t layer, const float *k, const float *v, size_t m) {
    return kv_push(kv, layer, k, v, m, hipMemcpyDeviceToDevice);
}

int kh_kv_len(const kh_kv *kv, size_t *len) {
    if (!kv || !len) return fail(KH_EINVAL, "kh_kv_len: null argument");
    *len = kv->len;
    return KH_OK;
}

int kh_kv_set_len(kh_kv *kv, size_t len) {
    if (!kv) return fail(KH_EINVAL, "kh_kv_set_len: null argument");
    kv->len = len;
    return KH_OK;
}

int kh_kv_truncate(kh_kv *kv, size_t len, size_t *kept) {
    if (!kv) return fail(KH_EINVAL, "kh_kv_truncate: null argument");
    if (len < kv->len) {
        for (size_t l = 0; l < kv->n_layer; l++)
            if (kv->rows[l] > len) kv->rows[l] = len;
        kv->len = len;
    }
    if (kept) *kept = kv->len;
    return KH_OK;
}

int kh_kv_clear(kh_kv *kv) {
    if (!kv) return fail(KH_EINVAL, "kh_kv_clear: null argument");
    for (size_t l = 0; l < kv->n_layer; l++) kv->rows[l] = 0;
    kv->len = 0;
    return KH_OK;
}

static int kv_read(const kh_kv *kv, size_t layer, bool keys, float *out, size_t *rows) {
    if (!kv) return fail(KH_EINVAL, "kh_kv_keys: null argument");
    if (layer >= kv->n_layer) return fail(KH_EINVAL, "kh_kv_keys: no such layer");
    Guard g(kv->ctx);
    size_t r = kv->rows[layer], dim = keys ? kv->k_dim : kv->v_dim;
    if (rows) *rows = r;
    if (out && r) {
        KH_HIP(hipMemcpyAsync(out, keys ? kv->k[layer] : kv->v[layer], 4 * r * dim, hipMemcpyDeviceToHost,
                              kv->ctx->stream));
        KH_HIP(hipStreamSynchronize(kv->ctx->stream));
    }
    return KH_OK;
}

int kh_kv_keys(const kh_kv *kv, size_t layer, float *out, size_t *rows) { return kv_read(kv, layer, true, out, rows); }

int kh_kv_values(const kh_kv *kv, size_t layer, float *out, size_t *rows) {
    return kv_read(kv, layer, false, out, rows);
}

int kh_kv_layer_ptrs(const kh_kv *kv, size_t layer, float **k, float **v) {
    if (!kv || layer >= kv->n_layer) return fail(KH_EINVAL, "kh_kv_layer_ptrs: bad argument");
    if (k) *k = kv->k[layer];
    if (v) *v = kv->v[layer];
    return KH_OK;
}

// ---- attention ---------------------------------------------------------------

int kh_attend_dev(kh_ctx *ctx, size_t n_head, size_t n_kv_head, size_t head_dim, const float *q, const float *k,
                  const float *v, size_t n_positions, float *out) {
    if (!ctx || !q || !out || (n_positions && (!k || !v))) return fail(KH_EINVAL, "kh_attend_dev: null argument");
    Guard g(ctx);
    size_t kv_dim = n_kv_head * head_dim;
    return launch_attend(ctx, (int)n_head, (int)n_kv_head, (int)head_dim, q, k, v, kv_dim, kv_dim, n_positions, out);
}

int kh_attend_dev_noalloc(kh_ctx *ctx, size_t n_head, size_t n_kv_head, size_t head_dim, const float *q,
                          const float *k, const float *v, size_t n_positions, float *out) {
    if (!ctx || !q || !out || (n_positions && (!k || !v))) return fail(KH_EINVAL, "kh_attend_dev_noalloc: null argument");
    Guard g(ctx);
    size_t kv_dim = n_kv_head * head_dim;
    return launch_attend_noalloc(ctx, (int)n_head, (int)n_kv_head, (int)head_dim, q, k, v, kv_dim, kv_dim,
                                 n_positions, out);
}

size_t kh_noalloc_scratch_bytes(void) { return scratch_bytes(); }

int kh_attend(kh_ctx *ctx, const kh_kv *kv, size_t layer, size_t n_head, size_t n_kv_head, size_t head_dim,
              const float *q, size_t n_positions, float *out) {
    if (!ctx || !kv || !q || !out) return fail(KH_EINVAL, "kh_attend: null argument");
    if (layer >= kv->n_layer) return fail(KH_EINVAL, "kh_attend: no such layer");
    if (kv->k_dim != n_kv_head * head_dim || kv->v_dim != n_kv_head * head_dim)
        return fail(KH_EINVAL, "kh_attend: cache width is not n_kv_head * head_dim");
    if (n_positions > kv->rows[layer]) return fail(KH_EINVAL, "kh_attend: more positions than the cache holds");
    Guard g(ctx);
    const size_t nq = n_head * head_dim;
    int rc = ensure(ctx, ctx->io, 2 * up(4 * nq));
    if (rc) return rc;
    float *dq = static_cast<float *>(ctx->io.ptr);
    float *dout = reinterpret_cast<float *>(static_cast<char *>(ctx->io.ptr) + up(4 * nq));
    KH_HIP(hipMemcpyAsync(dq, q, 4 * nq, hipMemcpyHostToDevice, ctx->stream));
    rc = launch_attend(ctx, (int)n_head, (int)n_kv_head, (int)head_dim, dq, kv->k[layer], kv->v[layer], kv->k_dim,
                       kv->v_dim, n_positions, dout);
    if (rc) return rc;
    KH_HIP(hipMemcpyAsync(out, dout, 4 * nq, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

// ---- latent attention (DeepSeek) ---------------------------------------------

int kh_mla_attend_dev(kh_ctx *ctx, size_t n_head, const float *q_lat, const float *q_pe, const float *c,
                      const float *pe, size_t n_positions, float scale, float *out) {
    if (!ctx || !q_lat || !q_pe || !out || (n_positions && (!c || !pe)))
        return fail(KH_EINVAL, "kh_mla_attend_dev: null argument");
    if (n_head == 0 || n_head > 4096) return fail(KH_EINVAL, "kh_mla_attend_dev: bad head count");
    Guard g(ctx);
    return launch_mla(ctx, (int)n_head, q_lat, q_pe, c, pe, 512, 64, n_positions, scale, out);
}

int kh_mla_attend(kh_ctx *ctx, const kh_kv *kv, size_t layer, size_t n_head, const float *q_lat, const float *q_pe,
                  size_t n_positions, float scale, float *out) {
    if (!ctx || !kv || !q_lat || !q_pe || !out) return fail(KH_EINVAL, "kh_mla_attend: null argument");
    if (layer >= kv->n_layer) return fail(KH_EINVAL, "kh_mla_attend: no such layer");
    if (kv->k_dim != 64 || kv->v_dim != 512)
        return fail(KH_DECLINED, "kh_mla_attend: the cache must hold rope keys of 64 and latents of 512");
    if (n_positions > kv->rows[layer]) return fail(KH_EINVAL, "kh_mla_attend: more positions than the cache holds");
    if (n_head == 0 || n_head > 4096) return fail(KH_EINVAL, "kh_mla_attend: bad head count");
    Guard g(ctx);
    const size_t nl = n_head * 512, np = n_head * 64;
    int rc = ensure(ctx, ctx->io, up(4 * nl) + up(4 * np) + up(4 * nl));
    if (rc) return rc;
    char *base = static_cast<char *>(ctx->io.ptr);
    float *dql = reinterpret_cast<float *>(base), *dqp = reinterpret_cast<float *>(base + up(4 * nl));
    float *dout = reinterpret_cast<float *>(base + up(4 * nl) + up(4 * np));
    KH_HIP(hipMemcpyAsync(dql, q_lat, 4 * nl, hipMemcpyHostToDevice, ctx->stream));
    KH_HIP(hipMemcpyAsync(dqp, q_pe, 4 * np, hipMemcpyHostToDevice, ctx->stream));
    rc = launch_mla(ctx, (int)n_head, dql, dqp, kv->v[layer], kv->k[layer], kv->v_dim, kv->k_dim, n_positions, scale,
                    dout);
    if (rc) return rc;
    KH_HIP(hipMemcpyAsync(out, dout, 4 * nl, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

// ---- mixture of experts ------------------------------------------------------

int kh_moe_new(kh_ctx *ctx, size_t n_experts, size_t top_k, size_t hidden, size_t inter, int scoring, int select,
               size_t n_group, size_t topk_group, int norm_topk, float scale, const float *bias, kh_moe **out) {
    if (!ctx || !out) return fail(KH_EINVAL, "kh_moe_new: null argument");
    *out = nullptr;
    if (n_experts == 0 || top_k == 0 || top_k > n_experts || hidden == 0 || inter == 0)
        return fail(KH_EINVAL, "kh_moe_new: needs experts, 0 < top_k <= experts, and widths");
    if (n_experts > 512 || top_k > 16 || n_group > 64)
        return fail(KH_DECLINED, "kh_moe_new: more than 512 experts, 16 picks or 64 groups");
    if (scoring < 0 || scoring > 1 || select < 0 || select > 2)
        return fail(KH_EINVAL, "kh_moe_new: unknown scoring or selection");
    if (n_group == 0 || n_experts % n_group != 0)
        return fail(KH_EINVAL, "kh_moe_new: experts must divide into n_group groups");
    Guard g(ctx);
    std::unique_ptr<kh_moe> m(new kh_moe());
    m->ctx = ctx;
    m->n_experts = n_experts;
    m->top_k = top_k;
    m->hidden = hidden;
    m->inter = inter;
    m->scoring = scoring;
    m->select = select;
    m->n_group = n_group;
    m->topk_group = topk_group;
    m->norm_topk = norm_topk;
    m->scale = scale;
    m->gate.assign(n_experts, nullptr);
    m->up.assign(n_experts, nullptr);
    m->down.assign(n_experts, nullptr);
    KH_HIP(hipMalloc(reinterpret_cast<void **>(&m->tab), sizeof(void *) * 3 * n_experts));
    KH_HIP(hipMalloc(reinterpret_cast<void **>(&m->stab), sizeof(float *) * 3 * n_experts));
    KH_HIP(hipMalloc(reinterpret_cast<void **>(&m->arrivals), sizeof(unsigned)));
    KH_HIP(hipMemset(m->arrivals, 0, sizeof(unsigned)));  // the decode step's router leaves it at zero
    if (bias) {
        KH_HIP(hipMalloc(reinterpret_cast<void **>(&m->bias), 4 * n_experts));
        KH_HIP(hipMemcpy(m->bias, bias, 4 * n_experts, hipMemcpyHostToDevice));
    }
    *out = m.release();
    return KH_OK;
}

int kh_moe_free(kh_moe *moe) {
    if (!moe) return KH_OK;
    {
        Guard g(moe->ctx);
        (void)hipStreamSynchronize(moe->ctx->stream);
        if (moe->tab) (void)hipFree(moe->tab);
        if (moe->stab) (void)hipFree(moe->stab);
        if (moe->arrivals) (void)hipFree(moe->arrivals);
        if (moe->bias) (void)hipFree(moe->bias);
    }
    delete moe;
    return KH_OK;
}

int kh_moe_set_router(kh_moe *moe, const kh_weight *router) {
    if (!moe || check_weight(router)) return fail(KH_EINVAL, "kh_moe_set_router: null argument");
    if (router->rows != moe->n_experts || router->cols != moe->hidden)
        return fail(KH_EINVAL, "kh_moe_set_router: the router is [n_experts, hidden]");
    moe->router = router;
    return KH_OK;
}

int kh_moe_set_expert(kh_moe *moe, size_t expert, const kh_weight *gate, const kh_weight *up,
                      const kh_weight *down) {
    if (!moe || check_weight(gate) || check_weight(up) || check_weight(down))
        return fail(KH_EINVAL, "kh_moe_set_expert: null argument");
    if (expert >= moe->n_experts) return fail(KH_EINVAL, "kh_moe_set_expert: no such expert");
    if (gate->rows != moe->inter || gate->cols != moe->hidden || up->rows != moe->inter ||
        up->cols != moe->hidden || down->rows != moe->hidden || down->cols != moe->inter)
        return fail(KH_EINVAL, "kh_moe_set_expert: gate/up are [inter, hidden], down [hidden, inter]");
    const int p = gate->precision;
    if (p == KH_F32 || up->precision != p || down->precision != p)
        return fail(KH_DECLINED, "kh_moe_set_expert: an expert's three weights must share one quantised precision");
    if (moe->precision >= 0 && moe->precision != p)
        return fail(KH_DECLINED, "kh_moe_set_expert: every expert must have the same precision");
    moe->precision = p;
    moe->gate[expert] = gate;
    moe->up[expert] = up;
    moe->down[expert] = down;
    moe->dirty = true;
    return KH_OK;
}

int kh_moe_set_shared(kh_moe *moe, const kh_weight *gate, const kh_weight *up, const kh_weight *down) {
    if (!moe || check_weight(gate) || check_weight(up) || check_weight(down))
        return fail(KH_EINVAL, "kh_moe_set_shared: null argument");
    if (gate->cols != moe->hidden || up->cols != moe->hidden || up->rows != gate->rows ||
        down->rows != moe->hidden || down->cols != gate->rows || gate->rows % BLOCK)
        return fail(KH_EINVAL, "kh_moe_set_shared: gate/up are [width, hidden], down [hidden, width]");
    if (gate->precision == KH_F32 || up->precision == KH_F32 || down->precision == KH_F32 ||
        gate->precision != up->precision)
        return fail(KH_DECLINED, "kh_moe_set_shared: the shared expert must be quantised");
    moe->sgate = gate;
    moe->sup = up;
    moe->sdown = down;
    return KH_OK;
}

int kh_moe_run_dev(kh_ctx *ctx, kh_moe *moe, const float *hs, size_t m, float *out) {
    if (!ctx || !moe || !hs || !out) return fail(KH_EINVAL, "kh_moe_run_dev: null argument");
    Guard g(ctx);
    return moe_run_device(ctx, moe, hs, m, out);
}

int kh_moe_run(kh_ctx *ctx, kh_moe *moe, const float *hs, size_t m, float *out) {
    if (!ctx || !moe || !hs || !out) return fail(KH_EINVAL, "kh_moe_run: null argument");
    if (m == 0) return KH_OK;
    Guard g(ctx);
    const size_t n = m * moe->hidden;
    int rc = ensure(ctx, ctx->io, 2 * up(4 * n));
    if (rc) return rc;
    float *dx = static_cast<float *>(ctx->io.ptr);
    float *dy = reinterpret_cast<float *>(static_cast<char *>(ctx->io.ptr) + up(4 * n));
    KH_HIP(hipMemcpyAsync(dx, hs, 4 * n, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = moe_run_device(ctx, moe, dx, m, dy))) return rc;
    KH_HIP(hipMemcpyAsync(out, dy, 4 * n, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

int kh_debug_moe_picks(kh_ctx *ctx, const kh_moe *moe, size_t m, const kh_moe_picks *out) {
    if (!ctx || !moe || !out) return fail(KH_EINVAL, "kh_debug_moe_picks: null argument");
    Guard g(ctx);
    MoePicks o{out->logits,  out->count,     out->experts, out->weights,     out->gate,      out->up,
               out->hidden_qs, out->hidden_scales, out->out, out->shared_gate, out->shared_up, out->shared_out};
    return moe_picks(ctx, moe, m, o);
}

int kh_moe_route(kh_ctx *ctx, const kh_moe *moe, const float *logits, size_t m, int32_t *experts, float *weights,
                 int32_t *count) {
    if (!ctx || !moe || !logits || !experts || !weights || !count) return fail(KH_EINVAL, "kh_moe_route: null argument");
    if (m == 0) return KH_OK;
    Guard g(ctx);
    const size_t nl = m * moe->n_experts, np = m * moe->top_k;
    int rc = ensure(ctx, ctx->io, up(4 * nl) + 2 * up(4 * np) + up(4 * m));
    if (rc) return rc;
    char *p = static_cast<char *>(ctx->io.ptr);
    float *dl = reinterpret_cast<float *>(p);
    int32_t *de = reinterpret_cast<int32_t *>(p + up(4 * nl));
    float *dw = reinterpret_cast<float *>(p + up(4 * nl) + up(4 * np));
    int32_t *dc = reinterpret_cast<int32_t *>(p + up(4 * nl) + 2 * up(4 * np));
    KH_HIP(hipMemcpyAsync(dl, logits, 4 * nl, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = route_device(ctx, moe, dl, m, de, dw, dc))) return rc;
    KH_HIP(hipMemcpyAsync(experts, de, 4 * np, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipMemcpyAsync(weights, dw, 4 * np, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipMemcpyAsync(count, dc, 4 * m, hipMemcpyDeviceToHost, ctx->stream));
    KH_HIP(hipStreamSynchronize(ctx->stream));
    return KH_OK;
}

}  // extern "C"
