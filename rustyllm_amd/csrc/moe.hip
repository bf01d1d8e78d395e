// moe.hip — the routed mixture-of-experts feed-forward block of gpt-oss
// decode (forward_gpt_oss_into, src/model.rs:6846-6898): router selection,
// the gpt-oss SwiGLU with expert biases, and the weighted combine.  The
// expert matrix-vector products are f32-activation GEMV launches (MXFP4 or
// Q8_0) whose expert is read on the device (GemvMat::sel), so a whole block
// runs without a host round trip.
#pragma once
#include "attention_exact.hip"  // expf_glibc
#include "common.hpp"

namespace rh {

// f32::total_cmp order as a signed integer key (negative values have every
// bit but the sign flipped, so -0.0 < +0.0 and NaNs sort by payload).
__device__ __forceinline__ int32_t total_key(float v) {
    const int32_t b = __builtin_bit_cast(int32_t, v);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

// select_top_logits_into + bubble_up_router_last (src/model.rs:6659-6716):
// inserting each logit in index order and moving it up only past strictly
// smaller ones keeps the k largest in total order, largest first, an earlier
// index first among equal ones; that is each logit's rank here.  Then
// softmax_selected_into (:6639-6656): m = max, e_r = exp(v_r - m), sum in
// slot order, e_r /= sum.  One wave; n <= 64 experts, k <= 8.
__device__ __forceinline__ void moe_topk_row(const float *logits, int n, int k, int32_t *sel, float *prob) {
    __shared__ float s_v[8];
    __shared__ int32_t s_i[8];
    const int lane = threadIdx.x;
    const float v = lane < n ? logits[lane] : 0.0f;
    const int32_t key = total_key(v);
    int rank = 0;
    for (int j = 0; j < n; j++) {
        const int32_t kj = __shfl(key, j, 64);
        rank += (kj > key || (kj == key && j < lane)) ? 1 : 0;
    }
    if (lane < n && rank < k) {
        s_v[rank] = v;
        s_i[rank] = lane;
    }
    __syncthreads();
    if (lane == 0) {
        float m = -INFINITY;
        for (int r = 0; r < k; r++) m = fmaxf(m, s_v[r]);  // f32::max keeps the non-NaN operand
        float e[8], sum = 0.0f;
        for (int r = 0; r < k; r++) {
            e[r] = expf_glibc(s_v[r] - m);
            sum += e[r];
        }
        for (int r = 0; r < k; r++) {
            sel[r] = s_i[r];
            prob[r] = sum > 0.0f ? e[r] / sum : e[r];
        }
    }
}

// moe_topk_row's selection inside a one-wave workgroup (no LDS, no
// workgroup barrier): returns the expert of slot `slot` (wave-uniform); with
// sel non-null lane 0 also stores every slot's expert and softmax weight,
// computed as moe_topk_row computes them.
__device__ __forceinline__ int moe_topk_wave(const float *logits, int n, int k, int slot, int32_t *sel, float *prob) {
    const int lane = threadIdx.x & 63;
    const float v = lane < n ? logits[lane] : 0.0f;
    const int32_t key = total_key(v);
    // rank = the number of lanes ahead of this one in (key descending, index
    // ascending) order; each key is broadcast by a scalar read of its lane
    int rank = 0;
    for (int j = 0; j < n; j++) {
        const int32_t kj = __builtin_amdgcn_readlane(key, j);
        rank += (kj > key || (kj == key && j < lane)) ? 1 : 0;
    }
    const unsigned long long ms = __builtin_amdgcn_ballot_w64(lane < n && rank == slot);
    const int e_slot = ms ? (int)__builtin_ctzll(ms) : 0;
    if (sel) {
        float vr[8];
        int ir[8];
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const unsigned long long m = __builtin_amdgcn_ballot_w64(lane < n && rank == r);
            ir[r] = m ? (int)__builtin_ctzll(m) : 0;
            vr[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), ir[r]));
        }
        if (lane == 0) {
            float mx = -INFINITY;
            for (int r = 0; r < k; r++) mx = fmaxf(mx, vr[r]);  // f32::max keeps the non-NaN operand
            float e[8], sum = 0.0f;
            for (int r = 0; r < k; r++) {
                e[r] = expf_glibc(vr[r] - mx);
                sum += e[r];
            }
            for (int r = 0; r < k; r++) {
                sel[r] = ir[r];
                prob[r] = sum > 0.0f ? e[r] / sum : e[r];
            }
        }
    }
    return e_slot;
}

__global__ __launch_bounds__(64) void moe_topk_kernel(const float *logits, int n, int k, int32_t *sel, float *prob) {
    moe_topk_row(logits, n, k, sel, prob);
}

// swiglu_gpt_oss (src/model.rs:6596-6600): min(g, 7) (a NaN g gives 7),
// clamp(u, -7, 7) (a NaN u stays NaN), g * (1 / (1 + exp(-1.702 g))) * (u + 1).
__device__ __forceinline__ float swiglu_gpt_oss_ref(float g, float u) {
    g = fminf(g, 7.0f);
    u = u < -7.0f ? -7.0f : (u > 7.0f ? 7.0f : u);
    return g * (1.0f / (1.0f + expf_glibc(-1.702f * g))) * (u + 1.0f);
}

// gate_r[i] = swiglu_gpt_oss(gate_r[i] + gb[e_r][i], up_r[i] + ub[e_r][i])
// for the k slots (src/model.rs:6880-6882); a null bias adds nothing.
__global__ __launch_bounds__(256) void moe_swiglu_kernel(float *gate, const float *up, int hidden, int k,
                                                         const int32_t *sel, const float *gb, int gb_stride,
                                                         const float *ub, int ub_stride) {
    const int i = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    if (i >= hidden || r >= k) return;
    const int e = sel[r];
    float g = gate[(size_t)r * hidden + i], u = up[(size_t)r * hidden + i];
    if (gb) g = g + gb[(size_t)e * gb_stride + i];
    if (ub) u = u + ub[(size_t)e * ub_stride + i];
    gate[(size_t)r * hidden + i] = swiglu_gpt_oss_ref(g, u);
}

// moe[i] = 0, then per slot in order moe[i] += (proj_r[i] + db[e_r][i]) * p_r
// (src/model.rs:6886-6890); x[i] += moe[i] when x is given (:6894-6896).
__global__ __launch_bounds__(256) void moe_combine_kernel(const float *proj, int dim, int k, const int32_t *sel,
                                                          const float *prob, const float *db, int db_stride,
                                                          float *moe, float *x) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= dim) return;
    float acc = 0.0f;
    for (int r = 0; r < k; r++) {
        float v = proj[(size_t)r * dim + i];
        if (db) v = v + db[(size_t)sel[r] * db_stride + i];
        acc += v * prob[r];
    }
    if (moe) moe[i] = acc;
    if (x) x[i] += acc;
}

}  // namespace rh
