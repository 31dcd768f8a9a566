// Device helpers shared by the GEMV kernels (gemv.hip, dequant.hip) and the
// session (session.hip): buffer loads, DPP lane moves, the wave sum, the
// Q4_K header decode and the dequantised weight element.
#pragma once

#include "common.hpp"

namespace kh {
namespace dev {

constexpr int WAVE = 64;
constexpr unsigned RSRC_WORD3 = 0x00020000;  // raw buffer, gfx9 family

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// A buffer descriptor over `bytes` bytes at p: loads past the end return 0.
__device__ __forceinline__ rsrc_t rsrc(const void *p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)(bytes > 0xffffffffu ? 0xffffffffu : bytes), RSRC_WORD3);
}
__device__ __forceinline__ int4 bld16(rsrc_t r, unsigned off) {
    return __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float4 bld16f(rsrc_t r, unsigned off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float bldf(rsrc_t r, unsigned off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ int bldi(rsrc_t r, unsigned off) {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// f32 read through the scalar cache (constant address space): for values a
// kernel only reads, at wave-uniform addresses.  Such loads are counted apart
// from vector loads, so they never wait for weight loads in flight.
typedef const __attribute__((address_space(4))) float const_f32;

// A pointer every lane holds alike, moved to scalar registers.
template <typename T>
__device__ __forceinline__ T *uniform_ptr(T *p) {
    const unsigned long long v = reinterpret_cast<unsigned long long>(p);
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return reinterpret_cast<T *>(((unsigned long long)hi << 32) | lo);
}

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// a * b for operands the caller knows to fit in 24 signed bits: one
// full-rate v_mul_i32_i24 (the compiler would otherwise mask the operands or
// use the quarter-rate 32-bit multiply).
__device__ __forceinline__ int mul24(int a, int b) {
    int r;
    asm("v_mul_i32_i24 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// DPP lane movement (gfx9 encodings): quad_perm [1,0,3,2] = xor 1,
// quad_perm [2,3,0,1] = xor 2, row_half_mirror, row_mirror.
template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __builtin_bit_cast(float, dpp<CTRL>(__builtin_bit_cast(int, v)));
}
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

// Sum over the wave; every lane gets the same value, in a fixed order.
__device__ __forceinline__ float wave_sum(float v) {
    v += dppf<DPP_XOR1>(v);
    v += dppf<DPP_XOR2>(v);
    v += dppf<DPP_HALF_MIRROR>(v);
    v += dppf<DPP_MIRROR>(v);
    float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (a + b) + (c + d);
}

// Xor over the wave (every lane gets it).
__device__ __forceinline__ unsigned wave_xor(unsigned v) {
    for (int o = WAVE / 2; o > 0; o >>= 1) v ^= (unsigned)__shfl_xor((int)v, o);
    return v;
}

__device__ __forceinline__ float half_bits_to_float(unsigned h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffff));
}

// The 6-bit scale and minimum of Q4_K sub-block j (mpp.rs:276-282) from
// bytes 4..15 of the block header (h.y, h.z, h.w), without a branch: j is
// fixed per lane, so sh = 8 (j & 3) and hij = (j >= 4 ? ~0 : 0) are lane
// constants.  For j < 4 this is A & 63 and B & 63; for j >= 4, the low four
// bits from byte 8 + j and the top two from bytes j and 4 + j.
__device__ __forceinline__ void q4k_scale_min(const int4 &h, int sh, unsigned hij, unsigned &sc, unsigned &mn) {
    const unsigned A = (unsigned)h.y >> sh, B = (unsigned)h.z >> sh, Cw = (unsigned)h.w >> sh;
    const unsigned s2 = hij & 2u;
    const unsigned X = A ^ ((A ^ Cw) & hij), Y = B ^ ((B ^ (Cw >> 4)) & hij);
    sc = (X & 0xfu) | ((A >> s2) & 0x30u);
    mn = (Y & 0xfu) | ((B >> s2) & 0x30u);
}

// Element k of row r of a weight, dequantised: Weight::row (quant.rs:374-402)
// for q8 ((f32)q * s) and q4 ((f32)(nibble - 8) * s), the Q4_K decoder
// (mpp.rs:304-315: (f32(d) * sc) * q - f32(dmin) * m), or the f32 value.
__device__ __forceinline__ float dequant_elem(int prec, const void *qs, const float *scales, size_t cols, size_t r,
                                              size_t k) {
    const size_t nb = cols / BLOCK;
    if (prec == KH_Q8) {
        const int8_t *q = static_cast<const int8_t *>(qs) + r * cols;
        return (float)q[k] * scales[r * nb + k / BLOCK];
    } else if (prec == KH_Q4) {
        const uint8_t *q = static_cast<const uint8_t *>(qs) + r * cols / 2;
        const size_t b = k / BLOCK, o = k % BLOCK;
        const uint8_t byte = q[b * 16 + (o & 15)];
        const int code = o < 16 ? (byte & 0x0f) : (byte >> 4);
        return (float)(code - 8) * scales[r * nb + b];
    } else if (prec == KH_Q4K) {
        const uint8_t *blk = static_cast<const uint8_t *>(qs) + (r * (cols / QK_K) + k / QK_K) * Q4K_BYTES;
        const int p = (int)(k % QK_K), j = p / 32, c = p / 64, h = (p / 32) & 1, l = p % 32;
        const uint8_t *s = blk + 4;
        int sc, mn;
        if (j < 4) {
            sc = s[j] & 63;
            mn = s[j + 4] & 63;
        } else {
            sc = (s[j + 4] & 0xf) | ((s[j - 4] >> 6) << 4);
            mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const float dl = half_bits_to_float(blk[0] | (blk[1] << 8)) * (float)sc;
        const float ml = half_bits_to_float(blk[2] | (blk[3] << 8)) * (float)mn;
        const int q = (blk[16 + 32 * c + l] >> (4 * h)) & 0xf;
        const float t = dl * (float)q;
        return t - ml;
    }
    return static_cast<const float *>(qs)[r * cols + k];
}

}  // namespace dev
}  // namespace kh
