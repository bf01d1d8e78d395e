// gemm_mfma.hip — batched K-quant matrix products on the matrix cores, for
// prefill: y[t][r] = row r of W times token t's Q8_K activation, the batch
// matvec of forward_prefill_batch (matvec_kquant3_batch_into,
// src/simd.rs:3461-3578).  Each (row, token) result is bit-identical to the
// single-token GEMV row: the per-block integer sums are exact, and the f32
// combine is the same expression in the same block order (as the reference's
// x4 kernels are bit-identical to its single-token dots, tests
// src/simd.rs:8540-8608).
//
// v_mfma_i32_32x32x32_i8 / _32x32x16_i8 lane layout (checked on gfx950):
// A[m = l%32][k = K8*(l/32) + j], B[k][n = l%32], C[i] at
// m = 8*(i/4) + 4*(l/32) + i%4, n = l%32, with K8 = 16 (x32) or 8 (x16).
// Here m = token and n = weight row: a lane owns one weight row, so its
// scales and minimums are per-lane values, and 16 tokens.
//   Q4_K: one x32 MFMA per 32-element sub-block on the raw nibbles (C_j =
//         sum q x exactly), isum += sc_j * C_j; imin = sum_j m_j * bsums_j =
//         sum_e m_j(e) * x_e is one more MFMA per sub-block with m_j as the
//         B operand; value = dx * (d*isum - dmin*imin).
//   Q6_K: one x16 MFMA per 16-element scale group on q - 32 as signed
//         bytes, isum += sc_g * C_g; value = (dx*d) * isum.
// Rows and tokens past the ends read clamped (in-bounds) data and are not
// stored.
#pragma once
#include "common.hpp"
#include "gemv.hip"

namespace rh {

typedef int rh_v4i __attribute__((ext_vector_type(4)));
typedef int rh_v16i __attribute__((ext_vector_type(16)));

struct GemmArgs {
    const uint8_t *w;
    int64_t row_stride;
    int32_t rows, K, T;
    int32_t epi;        // EPI_STORE or EPI_ADD
    const int8_t *xq;   // [T][K] Q8_K quants, token-major
    const float *dx;    // [K/256][ldx] Q8_K scales, token-minor
    int32_t ldx;        // >= T, a multiple of 4
    int32_t ldy;        // y[t * ldy + r]
    float *y;
    const float *bias;  // [rows] or null
};

#define GEMM_NT 2  // 32-token tiles per wave

// Q6_K bytes q (0..63, four per dword) as signed q - 32: flip bit 5, then copy
// it into bits 6 and 7.
__device__ __forceinline__ uint32_t q6_signed4(uint32_t q) {
    const uint32_t b = q ^ 0x20202020u, s = b & 0x20202020u;
    return b | (s << 1) | (s << 2);
}

template <int FMT>
__global__ __launch_bounds__(256) void gemm_kq_mfma_kernel(GemmArgs A) {
    const int lane = threadIdx.x & 63, half = lane >> 5, n = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r0 = (blockIdx.x * 4 + wave) * 32;
    if (r0 >= A.rows) return;  // whole-wave exit: no barrier follows
    const int t0 = blockIdx.y * 32 * GEMM_NT;
    const int row = min(r0 + n, A.rows - 1);
    const uint8_t *wr = A.w + (int64_t)row * A.row_stride;
    const int nb = A.K >> 8;
    // this lane's A-operand token per 32-token tile (clamped)
    const int8_t *xrow[GEMM_NT];
#pragma unroll
    for (int tt = 0; tt < GEMM_NT; tt++) xrow[tt] = A.xq + (int64_t)min(t0 + 32 * tt + n, A.T - 1) * A.K;
    float acc[GEMM_NT][16];
#pragma unroll
    for (int tt = 0; tt < GEMM_NT; tt++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[tt][i] = 0.0f;

    for (int b = 0; b < nb; b++) {
        int isum[GEMM_NT][16];
#pragma unroll
        for (int tt = 0; tt < GEMM_NT; tt++)
#pragma unroll
            for (int i = 0; i < 16; i++) isum[tt][i] = 0;
        float d, dmin = 0.0f;
        rh_v16i cmin[GEMM_NT];
        if (FMT == F_Q4_K) {
            const uint8_t *blk = wr + b * 144;
            const uint4 hdr = *(const uint4 *)blk;
            d = h2f(hdr.x & 0xFFFF);
            dmin = h2f(hdr.x >> 16);
#pragma unroll
            for (int tt = 0; tt < GEMM_NT; tt++) cmin[tt] = rh_v16i{};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint4 qs = *(const uint4 *)(blk + 16 + 32 * q + 16 * half);
                int sc0, m0, sc1, m1;
                scale_min_k4(2 * q, hdr.y, hdr.z, hdr.w, sc0, m0);
                scale_min_k4(2 * q + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
                const rh_v4i blo = {(int)(qs.x & 0x0F0F0F0Fu), (int)(qs.y & 0x0F0F0F0Fu), (int)(qs.z & 0x0F0F0F0Fu),
                                    (int)(qs.w & 0x0F0F0F0Fu)};
                const rh_v4i bhi = {(int)((qs.x >> 4) & 0x0F0F0F0Fu), (int)((qs.y >> 4) & 0x0F0F0F0Fu),
                                    (int)((qs.z >> 4) & 0x0F0F0F0Fu), (int)((qs.w >> 4) & 0x0F0F0F0Fu)};
                const int mb0 = m0 * 0x01010101, mb1 = m1 * 0x01010101;
                const rh_v4i bm0 = {mb0, mb0, mb0, mb0}, bm1 = {mb1, mb1, mb1, mb1};
#pragma unroll
                for (int tt = 0; tt < GEMM_NT; tt++) {
                    const rh_v4i a0 = *(const rh_v4i *)(xrow[tt] + 256 * b + 64 * q + 16 * half);
                    const rh_v4i a1 = *(const rh_v4i *)(xrow[tt] + 256 * b + 64 * q + 32 + 16 * half);
                    const rh_v16i c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, blo, rh_v16i{}, 0, 0, 0);
                    const rh_v16i c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bhi, rh_v16i{}, 0, 0, 0);
                    cmin[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bm0, cmin[tt], 0, 0, 0);
                    cmin[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bm1, cmin[tt], 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 16; i++) isum[tt][i] += __mul24(sc0, c0[i]) + __mul24(sc1, c1[i]);
                }
            }
        } else {
            const uint8_t *blk = wr + b * 210;
            d = ldh(blk + 208);
#pragma unroll
            for (int g = 0; g < 2; g++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    // qh bytes of positions 16h + 8*half .. +8 of half g
                    const uint2 qh = ld8(blk + 128 + 32 * g + 16 * h + 8 * half);
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const uint2 ql = ld8(blk + 64 * g + 32 * (k & 1) + 16 * h + 8 * half);
                        const int sh = 4 * (k >> 1);
                        const uint32_t q0 = ((ql.x >> sh) & 0x0F0F0F0Fu) | (((qh.x >> (2 * k)) & 0x03030303u) << 4);
                        const uint32_t q1 = ((ql.y >> sh) & 0x0F0F0F0Fu) | (((qh.y >> (2 * k)) & 0x03030303u) << 4);
                        const long bq = (long)((uint64_t)q6_signed4(q0) | ((uint64_t)q6_signed4(q1) << 32));
                        const int sc = (int)(int8_t)blk[192 + 8 * g + 2 * k + h];
                        const int e0 = 128 * g + 32 * k + 16 * h + 8 * half;
#pragma unroll
                        for (int tt = 0; tt < GEMM_NT; tt++) {
                            const long a = *(const long *)(xrow[tt] + 256 * b + e0);
                            const rh_v16i c = __builtin_amdgcn_mfma_i32_32x32x16_i8(a, bq, rh_v16i{}, 0, 0, 0);
#pragma unroll
                            for (int i = 0; i < 16; i++) isum[tt][i] += __mul24(sc, c[i]);
                        }
                    }
                }
        }
        // combine, block b: token m_i = 8*(i/4) + 4*half + i%4; dx of four
        // consecutive tokens per 16-byte load
#pragma unroll
        for (int tt = 0; tt < GEMM_NT; tt++) {
            const float *dxb = A.dx + (int64_t)b * A.ldx + t0 + 32 * tt + 4 * half;
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const float4 dv = *(const float4 *)(dxb + 8 * g4);
                const float dxs[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int i = 4 * g4 + r;
                    float v;
                    if (FMT == F_Q4_K) {
                        const float t1 = d * (float)isum[tt][i];
                        const float t2 = dmin * (float)cmin[tt][i];
                        v = dxs[r] * (t1 - t2);
                    } else {
                        v = (dxs[r] * d) * (float)isum[tt][i];
                    }
                    acc[tt][i] += v;
                }
            }
        }
    }
    if (r0 + n >= A.rows) return;
    const float bias = A.bias ? A.bias[r0 + n] : 0.0f;
#pragma unroll
    for (int tt = 0; tt < GEMM_NT; tt++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int t = t0 + 32 * tt + 8 * (i >> 2) + 4 * half + (i & 3);
            if (t >= A.T) continue;
            float *yp = A.y + (int64_t)t * A.ldy + r0 + n;
            float v = acc[tt][i];
            if (A.bias) v = v + bias;
            if (A.epi == EPI_ADD)
                *yp += v;
            else
                *yp = v;
        }
}

}  // namespace rh
