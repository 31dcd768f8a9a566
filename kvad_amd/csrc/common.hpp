// Internal declarations shared by the HIP translation units of libkvad_hip.
// Nothing here is part of the C ABI (include/kvad_hip.h is).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <mutex>
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
    kh::Workspace counters;  // zeroed once; kernels that use them leave them zero
};

struct kh_weight {
    kh_ctx *ctx = nullptr;
    int precision = 0;  // KH_F32 / KH_Q8 / KH_Q4 / KH_Q4K
    size_t rows = 0, cols = 0;
    void *qs = nullptr;        // q8: int8[rows*cols]; q4: uint8[rows*cols/2]; q4k: blocks; f32: float[rows*cols]
    float *scales = nullptr;   // q8/q4: float[rows*cols/32]
    size_t bytes = 0;          // bytes held on the device
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
    int rows;
    int cols;
    int wave0;              // set by the launcher: first workgroup of the job
    int nwaves;             // set by the launcher: waves working on the job
};

// Runs every job in one launch (all jobs share `precision`).
int launch_gemv(kh_ctx *ctx, int precision, const GemvJob *jobs, int njobs);

// Batched prefill y[m, rows] = xs[m, cols] W^T (+bias), m > 1 (device pointers).
int launch_matmul(kh_ctx *ctx, const kh_weight *w, const float *xs, size_t m, const float *bias, float *y);

// Split decode attention over one layer's cache, device pointers.
int launch_attend(kh_ctx *ctx, int n_head, int n_kv_head, int head_dim, const float *q, const float *k,
                  const float *v, size_t kv_stride_k, size_t kv_stride_v, size_t n_positions, float *out);

// Weight::quantize on device f32 data into qs/scales (scales unused for Q4_K).
int launch_quantize(kh_ctx *ctx, const float *w, size_t rows, size_t cols, int precision, void *qs, float *scales);

// Small helpers.
int launch_fill(kh_ctx *ctx, float *p, size_t n, float value);
int launch_dequant_row(kh_ctx *ctx, const kh_weight *w, size_t r, float *out);

}  // namespace kh
