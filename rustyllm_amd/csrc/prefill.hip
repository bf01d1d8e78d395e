// prefill.hip — the per-token steps of batched prefill (forward_prefill_batch,
// src/model.rs:9917-10090) for T tokens in one launch, token = blockIdx.y.
// Each is the decode step's arithmetic applied to every token row, and each
// ends in the Q8_K quantization the next batched product reads:
//   quants [T][K] (token-major) and scales [K/256][ldx] (token-minor).
#pragma once
#include "attention_exact.hip"
#include "common.hpp"
#include "gemv.hip"  // silu_mul_ref
#include "ops.hip"   // sumsq_avx2_order, dequant_elem

namespace rh {

// Q8_K of element e (0..255) of block b of token t, one element per thread
// (quantize_row_q8k, src/simd.rs:5013-5101; same arithmetic as
// q8k_block_store).
__device__ __forceinline__ void q8k_batch_store(float v, int b, int t, int K, int8_t *qs, float *dx, int ldx,
                                                float *red) {
    const float amax = block_max_256(fabsf(v), red);
    const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
    int q = (int)__builtin_rintf(v * id);
    q = max(-128, min(127, q));
    qs[(int64_t)t * K + b * 256 + threadIdx.x] = (int8_t)q;
    if (threadIdx.x == 0) dx[(int64_t)b * ldx + t] = amax * (1.0f / 127.0f);
}

// x [T][ldxf] -> Q8_K.  grid (K/256, T).
__global__ __launch_bounds__(256) void quantize_q8k_batch_kernel(const float *x, int K, int ldxf, int8_t *qs,
                                                                 float *dx, int ldx) {
    __shared__ float red[4];
    const int b = blockIdx.x, t = blockIdx.y;
    const float v = x[(int64_t)t * ldxf + b * 256 + threadIdx.x];
    q8k_batch_store(v, b, t, K, qs, dx, ldx, red);
}

// rms_norm_slice_into (src/model.rs:9889-9897, the same arithmetic as
// rms_norm_into): each token row of x [T][n] normalized with w, then Q8_K.
// One workgroup per token: the row's sum of squares once, in the reference's
// order, then wave w quantizes blocks w, w + 4, ... (four elements per lane;
// the block maximum is exact in any order, so the values are
// q8k_batch_store's).  n a multiple of 256.  grid (T), dynamic LDS n floats.
__global__ __launch_bounds__(256) void rmsnorm_q8k_batch_kernel(const float *x, const float *w, float eps, int n,
                                                                int8_t *qs, float *dx, int ldx) {
    extern __shared__ float s_x[];
    __shared__ float red[40];
    const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float *xr = x + (int64_t)t * n;
    for (int i = threadIdx.x; i < (n >> 2); i += 256) ((float4 *)s_x)[i] = ((const float4 *)xr)[i];
    __syncthreads();
    const float ss = sumsq_avx2_order(s_x, n, red);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (int b = wave; b < (n >> 8); b += 4) {
        const int e = 256 * b + 4 * lane;
        const float4 xv = *(const float4 *)(s_x + e), wv = *(const float4 *)(w + e);
        const float o[4] = {xv.x * scale * wv.x, xv.y * scale * wv.y, xv.z * scale * wv.z, xv.w * scale * wv.w};
        const float amax = wave_max(fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3]))));
        const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
        uint32_t packed = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int q = (int)__builtin_rintf(o[i] * id);
            q = max(-128, min(127, q));
            packed |= (uint32_t)(q & 0xFF) << (8 * i);
        }
        *(uint32_t *)(qs + (int64_t)t * n + e) = packed;
        if (lane == 0) dx[(int64_t)b * ldx + t] = amax * (1.0f / 127.0f);
    }
}

// silu_mul_into over the batch (src/model.rs:10071-10075): h = silu(g) * u
// with the reference's vector exp, then Q8_K for the down projection.
// grid (n/256, T).
__global__ __launch_bounds__(256) void silu_mul_q8k_batch_kernel(const float *gate, const float *up, int n,
                                                                 int8_t *qs, float *dx, int ldx) {
    __shared__ float red[4];
    const int t = blockIdx.y;
    const int64_t i = (int64_t)t * n + blockIdx.x * 256 + threadIdx.x;
    q8k_batch_store(silu_mul_ref(gate[i], up[i]), blockIdx.x, t, n, qs, dx, ldx, red);
}

// Final attention scale of every token (out * (1/den) where den > 0, as
// attn_exact_finish_kernel) and Q8_K of the rows for the output projection.
// out [T][n], token t's denominators at den + t*den_tok.  grid (n/256, T).
__global__ __launch_bounds__(256) void attn_finish_q8k_batch_kernel(const float *out, const float *den,
                                                                    int64_t den_tok, int vd, int n, int8_t *qs,
                                                                    float *dx, int ldx) {
    __shared__ float red[4];
    const int t = blockIdx.y, e = blockIdx.x * 256 + threadIdx.x;
    float v = out[(int64_t)t * n + e];
    const float d = den[(int64_t)t * den_tok + e / vd];
    if (d > 0.0f) {
        const float inv = 1.0f / d;
        v = v * inv;
    }
    q8k_batch_store(v, blockIdx.x, t, n, qs, dx, ldx, red);
}

// Embedding rows of T tokens (token_embd.row_into, src/model.rs:267-289).
// grid (ceil(dim/256), T).
__global__ __launch_bounds__(256) void embed_batch_kernel(const uint8_t *w, int64_t row_stride, int fmt, int dim,
                                                          const int32_t *tokens, float *x) {
    const int t = blockIdx.y, e = blockIdx.x * 256 + threadIdx.x;
    if (e >= dim) return;
    x[(int64_t)t * dim + e] = dequant_elem(w + (int64_t)tokens[t] * row_stride, fmt, e);
}

}  // namespace rh
