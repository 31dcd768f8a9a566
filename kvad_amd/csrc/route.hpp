// Router::route (crates/llm/src/model/ffn.rs:256-349) for one token on one
// wave: the MoE router kernel (moe.hip) runs it per token, and the decode
// step's router GEMV (gemv.hip) runs it in the workgroup that computed the
// token's logits, so the picks need no launch of their own.
#pragma once

#include "common.hpp"

namespace kh {
namespace {

constexpr int MAX_EXPERTS = 512;
constexpr int MAX_TOPK = 16;
constexpr int MAX_GROUPS = 64;

// The calling wave's LDS writes are complete before any of its later LDS
// reads (one wave: its lanes run in step, so no barrier is needed).
__device__ __forceinline__ void wave_lds_sync() { __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// f32::total_cmp as an integer key (-0.0 < +0.0; a total order).
__device__ __forceinline__ int total_key(float f) {
    const int b = __builtin_bit_cast(int, f);
    return b ^ (int)(((unsigned)(b >> 31)) >> 1);
}

// Router::route for one token, run by one wave (ffn.rs:256-309), over the
// token's logits `lg` (global memory or LDS).  The softmax's sum runs in one
// lane in index order and the picks' normalising total in pick order, as the
// reference sums them; the top-k picks the largest choice, the lowest index
// on ties.  Only the calling wave takes part: it syncs with itself
// (wave_lds_sync), never with the rest of its workgroup.
__device__ __forceinline__ void route_one(const RouteArgs &r, int tok, const float *lg) {
    const int lane = threadIdx.x & 63, n = r.n;
    __shared__ __align__(16) float s_score[MAX_EXPERTS], s_choice[MAX_EXPERTS];  // padded to n16
    __shared__ float s_inv;
    __shared__ int s_order[MAX_GROUPS];
    __shared__ float s_str[MAX_GROUPS];
    __shared__ int s_pick_e[MAX_TOPK];
    __shared__ float s_pick_w[MAX_TOPK];
    __shared__ int s_best;
    // Serial loops over the experts read 16 values at a time (four 16-byte
    // LDS reads in flight) and then use them in index order: one LDS round
    // trip per 16 experts rather than per expert.  Padding past n reads as
    // 0 (adding 0.0f to a positive sum is exact) or -inf (never a choice).
    const int n16 = (n + 15) & ~15;
    auto batch = [&](const float *a, int i0, float (&v)[16]) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = reinterpret_cast<const float4 *>(a + i0)[q];
            v[4 * q] = f.x, v[4 * q + 1] = f.y, v[4 * q + 2] = f.z, v[4 * q + 3] = f.w;
        }
    };

    if (r.scoring == 0) {  // softmax_inplace (tensor.rs:297-308)
        float mx = -INFINITY;
        for (int i = lane; i < n; i += 64) mx = fmaxf(mx, lg[i]);
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        for (int i = lane; i < n16; i += 64) s_score[i] = i < n ? expf(lg[i] - mx) : 0.0f;
        wave_lds_sync();
        if (lane == 0) {  // summed in index order, as the reference does
            float sum = 0.0f;
            for (int i0 = 0; i0 < n16; i0 += 16) {
                float v[16];
                batch(s_score, i0, v);
#pragma unroll
                for (int t = 0; t < 16; t++) sum += v[t];
            }
            s_inv = 1.0f / sum;
        }
        wave_lds_sync();
        for (int i = lane; i < n; i += 64) s_score[i] *= s_inv;
    } else {  // sigmoid (ffn.rs:262-266)
        for (int i = lane; i < n; i += 64) s_score[i] = 1.0f / (1.0f + expf(-lg[i]));
    }
    wave_lds_sync();
    for (int i = lane; i < n16; i += 64)
        s_choice[i] = i >= n ? -INFINITY : r.bias ? s_score[i] + r.bias[i] : s_score[i];
    wave_lds_sync();

    // mask_to_best_groups (ffn.rs:312-349)
    if (r.select != 0 && r.n_group > 1) {
        const int per = n / r.n_group;
        if (lane < r.n_group) {
            const float *grp = s_choice + lane * per;
            float st;
            if (r.select == 1) {
                st = -INFINITY;
                for (int i = 0; i < per; i++) st = fmaxf(st, grp[i]);
            } else {
                float a = -INFINITY, b = -INFINITY;
                for (int i = 0; i < per; i++) {
                    const float v = grp[i];
                    if (v > a) {
                        b = a;
                        a = v;
                    } else if (v > b) {
                        b = v;
                    }
                }
                st = a + b;
            }
            s_str[lane] = st;
        }
        wave_lds_sync();
        if (lane == 0) {  // stable sort, descending by total_cmp
            for (int g = 0; g < r.n_group; g++) s_order[g] = g;
            for (int i = 1; i < r.n_group; i++) {
                const int x = s_order[i];
                int j = i;
                while (j > 0 && total_key(s_str[s_order[j - 1]]) < total_key(s_str[x])) {
                    s_order[j] = s_order[j - 1];
                    j--;
                }
                s_order[j] = x;
            }
        }
        wave_lds_sync();
        const int keep = r.topk_group < r.n_group ? r.topk_group : r.n_group;
        for (int o = keep; o < r.n_group; o++)
            for (int i = lane; i < per; i += 64) s_choice[s_order[o] * per + i] = -INFINITY;
        wave_lds_sync();
    }

    // the picks (ffn.rs:279-293): the reference takes the largest choice,
    // the lowest index on ties, until top_k are taken or none is left; that
    // is the order of each valid expert's rank among the valid choices
    const int k = r.top_k < n ? r.top_k : n;
    if (lane == 0) s_best = 0;
    wave_lds_sync();
    for (int i = lane; i < n; i += 64) {
        const float v = s_choice[i];
        if (!(v > -INFINITY)) continue;
        int rank = 0;
        for (int j0 = 0; j0 < n16; j0 += 16) {
            float u[16];
            batch(s_choice, j0, u);
#pragma unroll
            for (int t = 0; t < 16; t++) rank += u[t] > -INFINITY && (u[t] > v || (u[t] == v && j0 + t < i));
        }
        if (rank < k) {
            s_pick_e[rank] = i;
            s_pick_w[rank] = s_score[i];
            atomicAdd(&s_best, 1);
        }
    }
    wave_lds_sync();
    const int got = __builtin_amdgcn_readfirstlane(s_best);  // the same in every lane

    // Lane i holds pick i.  The normalising total is summed in pick order
    // (one lane's values read across, as the reference adds them), each
    // pick's divide and scale are its own lane's, and every lane writes its
    // own slots.
    const bool mine = lane < got;
    const int pe = mine ? s_pick_e[lane] : 0;
    float pw = mine ? s_pick_w[lane] : 0.0f;
    const bool normalised = r.norm_topk && r.top_k > 1;
    if (normalised) {  // ffn.rs:296-302
        float total = 0.0f;
        for (int i = 0; i < got; i++)
            total += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pw), i));
        total += 1e-20f;
        pw = pw / total;
    }
    if (r.always_scale || !normalised) pw *= r.scale;
    if (lane < r.top_k) {
        r.experts[(size_t)tok * r.top_k + lane] = mine ? pe : -1;
        r.weights[(size_t)tok * r.top_k + lane] = mine ? pw : 0.0f;
    }
    if (lane == 0) r.count[tok] = got;
    if (r.sorted_experts) {
        // the picks in expert order (each pick's place is the number of
        // picks naming a smaller expert; the experts are distinct); unused
        // slots name expert 0 with weight 0, so a kernel that reads every
        // slot stays in bounds
        int at = 0;
        for (int i = 0; i < got; i++) at += __builtin_amdgcn_readlane(pe, i) < pe;
        const size_t o = (size_t)tok * r.top_k;
        if (mine) {
            r.sorted_experts[o + at] = pe;
            r.sorted_weights[o + at] = pw;
        } else if (lane < r.top_k) {
            r.sorted_experts[o + lane] = 0;
            r.sorted_weights[o + lane] = 0.0f;
        }
    }
}

}  // namespace
}  // namespace kh
