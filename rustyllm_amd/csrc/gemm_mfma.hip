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
//   Q4_K: two x32 MFMAs per 32-element sub-block on the nibbles times the
//         two base-8 digits of the sub-block scale, accumulated over the
//         block, so isum = sum_j sc_j * C_j (C_j = sum q x) exactly; imin =
//         sum_j m_j * bsums_j = sum_e m_j(e) * x_e is one more MFMA per
//         sub-block with m_j as the B operand; value = dx * (d*isum -
//         dmin*imin).
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

// Q6_K bytes q (0..63, four per dword) as signed q - 32: (q + 0x60) ^ 0x80
// per byte, where q + 0x60 <= 0x9F never carries into the next byte (one add
// and one xor per dword; a copy of bit 5 into bits 6 and 7 compiled to a
// quarter-rate multiply by 6).
__device__ __forceinline__ uint32_t q6_signed4(uint32_t q) { return (q + 0x60606060u) ^ 0x80808080u; }

// Byte m (< 256) in all four bytes of a dword (one v_perm_b32).
__device__ __forceinline__ int bcast_byte(int m) { return (int)__builtin_amdgcn_perm(0u, (uint32_t)m, 0u); }

// One block of the lane's weight row, as the lane's MFMA B operands need it
// (lane half h = lane / 32 takes k = 16h.. of each 32-element Q4_K sub-block,
// k = 8h.. of each 16-element Q6_K group).
template <int FMT>
struct GemmW;
template <>
struct GemmW<F_Q4_K> {
    uint4 hdr, qs[4];
};
template <>
struct GemmW<F_Q6_K> {
    uint2 ql[8], qh[4];
    uint4 sc;
    uint32_t d;
};

__device__ __forceinline__ void gemm_w_load(GemmW<F_Q4_K> &W, const uint8_t *blk, int half) {
    W.hdr = *(const uint4 *)blk;  // 144-byte blocks of 16-aligned rows
#pragma unroll
    for (int q = 0; q < 4; q++) W.qs[q] = *(const uint4 *)(blk + 16 + 32 * q + 16 * half);
}
__device__ __forceinline__ void gemm_w_load(GemmW<F_Q6_K> &W, const uint8_t *blk, int half) {
#pragma unroll
    for (int g = 0; g < 2; g++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            W.qh[2 * g + h] = ld8(blk + 128 + 32 * g + 16 * h + 8 * half);
#pragma unroll
            for (int kk = 0; kk < 2; kk++) W.ql[4 * g + 2 * h + kk] = ld8(blk + 64 * g + 32 * kk + 16 * h + 8 * half);
        }
    W.sc = ld16(blk + 192);
    W.d = ld2(blk + 208);
}

// LDS activation tile: one block (256 quants) of each of the workgroup's
// tokens, rows padded to 272 bytes so the 32 token rows one MFMA operand read
// touches start 4 banks apart.
#define GEMM_XS 272

// Integer sums of block b for the wave's 32 rows x 32*NT tokens: isum (and
// for Q4_K imin) per C element, from the activation tile xs.
typedef unsigned short rh_u16x2 __attribute__((ext_vector_type(2)));

// Each byte of the four dwords of x (nibbles, < 16) times s (< 8): one packed
// 16-bit multiply per dword, exact because no byte product (< 128) carries
// into the next byte.
__device__ __forceinline__ rh_v4i bytes_times(const rh_v4i &x, int s) {
    const rh_u16x2 m = {(unsigned short)s, (unsigned short)s};
    rh_v4i r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int xi = x[i];  // a plain int (a bit-cast of the element expression itself reads element 0)
        r[i] = __builtin_bit_cast(int, __builtin_bit_cast(rh_u16x2, xi) * m);
    }
    return r;
}

// Q4_K: the sub-block scale (6 bits) enters the B operand as two digits, sc
// = 8 * (sc >> 3) + (sc & 7), each digit times a nibble fitting a signed
// byte, so that the MFMAs accumulate the whole block: isum = 8 * hi + lo =
// sum_j sc_j * C_j exactly (the same integer as one MFMA per sub-block scaled
// afterwards, with no per-sub-block multiply-add on the vector ALU).
template <int NT>
__device__ __forceinline__ void gemm_block_ints(const GemmW<F_Q4_K> &W, const int8_t *xs, int lane,
                                                int (&isum)[NT][16], rh_v16i (&imin)[NT]) {
    const int half = lane >> 5, n = lane & 31;
    rh_v16i ahi[NT], alo[NT];
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
        imin[tt] = rh_v16i{};
        ahi[tt] = rh_v16i{};
        alo[tt] = rh_v16i{};
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
        int sc0, m0, sc1, m1;
        scale_min_k4(2 * q, W.hdr.y, W.hdr.z, W.hdr.w, sc0, m0);
        scale_min_k4(2 * q + 1, W.hdr.y, W.hdr.z, W.hdr.w, sc1, m1);
        const uint4 qs = W.qs[q];
        const rh_v4i blo = {(int)(qs.x & 0x0F0F0F0Fu), (int)(qs.y & 0x0F0F0F0Fu), (int)(qs.z & 0x0F0F0F0Fu),
                            (int)(qs.w & 0x0F0F0F0Fu)};
        const rh_v4i bhi = {(int)((qs.x >> 4) & 0x0F0F0F0Fu), (int)((qs.y >> 4) & 0x0F0F0F0Fu),
                            (int)((qs.z >> 4) & 0x0F0F0F0Fu), (int)((qs.w >> 4) & 0x0F0F0F0Fu)};
        const rh_v4i l8 = bytes_times(blo, sc0 >> 3), l1 = bytes_times(blo, sc0 & 7);
        const rh_v4i h8 = bytes_times(bhi, sc1 >> 3), h1 = bytes_times(bhi, sc1 & 7);
        const int mb0 = bcast_byte(m0), mb1 = bcast_byte(m1);
        const rh_v4i bm0 = {mb0, mb0, mb0, mb0}, bm1 = {mb1, mb1, mb1, mb1};
#pragma unroll
        for (int tt = 0; tt < NT; tt++) {
            const int8_t *xr = xs + (32 * tt + n) * GEMM_XS + 64 * q + 16 * half;
            const rh_v4i a0 = *(const rh_v4i *)xr;
            const rh_v4i a1 = *(const rh_v4i *)(xr + 32);
            ahi[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, l8, ahi[tt], 0, 0, 0);
            alo[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, l1, alo[tt], 0, 0, 0);
            imin[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bm0, imin[tt], 0, 0, 0);
            ahi[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, h8, ahi[tt], 0, 0, 0);
            alo[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, h1, alo[tt], 0, 0, 0);
            imin[tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bm1, imin[tt], 0, 0, 0);
        }
    }
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
#pragma unroll
        for (int i = 0; i < 16; i++) isum[tt][i] = (ahi[tt][i] << 3) + alo[tt][i];
}

template <int NT>
__device__ __forceinline__ void gemm_block_ints(const GemmW<F_Q6_K> &W, const int8_t *xs, int lane,
                                                int (&isum)[NT][16], rh_v16i (&imin)[NT]) {
    const int half = lane >> 5, n = lane & 31;
    (void)imin;
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
#pragma unroll
        for (int i = 0; i < 16; i++) isum[tt][i] = 0;
    const uint32_t scw[4] = {W.sc.x, W.sc.y, W.sc.z, W.sc.w};
#pragma unroll
    for (int g = 0; g < 2; g++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint2 qh = W.qh[2 * g + h];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint2 ql = W.ql[4 * g + 2 * h + (k & 1)];
                const int sh = 4 * (k >> 1);
                const uint32_t q0 = ((ql.x >> sh) & 0x0F0F0F0Fu) | (((qh.x >> (2 * k)) & 0x03030303u) << 4);
                const uint32_t q1 = ((ql.y >> sh) & 0x0F0F0F0Fu) | (((qh.y >> (2 * k)) & 0x03030303u) << 4);
                const long bq = (long)((uint64_t)q6_signed4(q0) | ((uint64_t)q6_signed4(q1) << 32));
                const int si = 8 * g + 2 * k + h;  // scale of 16-element group (g, k, h)
                const int sc = (int)(int8_t)(scw[si >> 2] >> (8 * (si & 3)));
                const int e0 = 128 * g + 32 * k + 16 * h + 8 * half;
#pragma unroll
                for (int tt = 0; tt < NT; tt++) {
                    const long a = *(const long *)(xs + (32 * tt + n) * GEMM_XS + e0);
                    const rh_v16i c = __builtin_amdgcn_mfma_i32_32x32x16_i8(a, bq, rh_v16i{}, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        isum[tt][i] = __mul24(sc, c[i]) + isum[tt][i];
                        // opaque to the optimiser: keeps one 24-bit multiply-add per
                        // update instead of products paired into three-input adds
                        asm("" : "+v"(isum[tt][i]));
                    }
                }
            }
        }
}

// Workgroup: 4 waves x 32 weight rows, 32*NT tokens.  Per block: the next
// block's weights (registers) and activation tile (registers, then the other
// LDS buffer) are loaded while this block's MFMAs and combine run; one
// barrier per block.  Waves past the last row compute clamped rows and store
// nothing, so every wave reaches every barrier.
template <int FMT, int NT>
__global__ __launch_bounds__(256) void gemm_kq_mfma_kernel(GemmArgs A) {
    extern __shared__ __align__(16) int8_t s_xs[];  // [2][32*NT][GEMM_XS]
    constexpr int TOK = 32 * NT;
    constexpr int NLD = TOK * 16 / 256;  // 16-byte activation pieces per thread per block
    const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, n = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r0 = (blockIdx.x * 4 + wave) * 32;
    const int t0 = blockIdx.y * TOK;
    const int row = min(r0 + n, A.rows - 1);
    const uint8_t *wr = A.w + (int64_t)row * A.row_stride;
    const int nb = A.K >> 8;
    constexpr int BB = FMT == F_Q4_K ? 144 : 210;
    // activation pieces: thread -> (token, 16-byte part)
    const int8_t *xsrc[NLD];
    int xdst[NLD];
#pragma unroll
    for (int j = 0; j < NLD; j++) {
        const int p = tid + 256 * j, tok = p >> 4, part = p & 15;
        xsrc[j] = A.xq + (int64_t)min(t0 + tok, A.T - 1) * A.K + 16 * part;
        xdst[j] = tok * GEMM_XS + 16 * part;
    }
    GemmW<FMT> W;
    gemm_w_load(W, wr, half);
    {
        uint4 st[NLD];
#pragma unroll
        for (int j = 0; j < NLD; j++) st[j] = *(const uint4 *)xsrc[j];
#pragma unroll
        for (int j = 0; j < NLD; j++) *(uint4 *)(s_xs + xdst[j]) = st[j];
    }
    __syncthreads();
    float acc[NT][16];
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[tt][i] = 0.0f;

    for (int b = 0; b < nb; b++) {
        const bool more = b + 1 < nb;
        const int bn = more ? b + 1 : b;
        GemmW<FMT> Wn;
        gemm_w_load(Wn, wr + (int64_t)bn * BB, half);
        uint4 st[NLD];
#pragma unroll
        for (int j = 0; j < NLD; j++) st[j] = *(const uint4 *)(xsrc[j] + 256 * bn);
        // this block's activation scales, four consecutive tokens per load:
        // token of C element i = 8*(i/4) + 4*half + i%4
        float4 dv[NT][4];
#pragma unroll
        for (int tt = 0; tt < NT; tt++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++)
                dv[tt][g4] = *(const float4 *)(A.dx + (int64_t)b * A.ldx + t0 + 32 * tt + 4 * half + 8 * g4);
        int isum[NT][16];
        rh_v16i imin[NT];
        gemm_block_ints<NT>(W, s_xs + (b & 1) * TOK * GEMM_XS, lane, isum, imin);
        float d, dmin = 0.0f;
        if constexpr (FMT == F_Q4_K) {
            d = h2f(W.hdr.x & 0xFFFF);
            dmin = h2f(W.hdr.x >> 16);
        } else {
            d = h2f(W.d & 0xFFFF);
        }
        // the reference's per-block combine, accumulated in block order
#pragma unroll
        for (int tt = 0; tt < NT; tt++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const float dxs[4] = {dv[tt][g4].x, dv[tt][g4].y, dv[tt][g4].z, dv[tt][g4].w};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int i = 4 * g4 + r;
                    float v;
                    if constexpr (FMT == F_Q4_K) {
                        const float t1 = d * (float)isum[tt][i];
                        const float t2 = dmin * (float)imin[tt][i];
                        v = dxs[r] * (t1 - t2);
                    } else {
                        v = (dxs[r] * d) * (float)isum[tt][i];
                    }
                    acc[tt][i] += v;
                }
            }
        if (more) {
#pragma unroll
            for (int j = 0; j < NLD; j++) *(uint4 *)(s_xs + ((b + 1) & 1) * TOK * GEMM_XS + xdst[j]) = st[j];
        }
        __syncthreads();
        W = Wn;
    }
    if (r0 + n >= A.rows) return;
    const float bias = A.bias ? A.bias[r0 + n] : 0.0f;
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
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

// The same products with the blocks of K split over the workgroup's four
// waves, for launches with too few (row tile, token tile) pairs to fill the
// chip (the q/k/v/o projections, the long-K down projection): one workgroup
// per 32 weight rows x 32 tokens, wave w computing blocks w, w+4, w+8, ...
// Each wave stages its own block's activations in its own LDS tile, computes
// the block's per-output value exactly as gemm_kq_mfma_kernel does, and
// leaves the 16 values of each lane in LDS; after a barrier, wave w adds the
// round's values of C elements 4w..4w+3 to its accumulators in block order
// (a barrier before the next round's values are written keeps them until
// every wave has read these).  Every output is therefore the same sum of
// the same per-block values in the same order: bit-identical to the
// one-wave-per-row-tile kernel.
template <int FMT>
__global__ __launch_bounds__(256) void gemm_kq_mfma_ks_kernel(GemmArgs A) {
    __shared__ __align__(16) int8_t s_xs[4][32 * GEMM_XS];  // per wave: 32 token rows of one block
    __shared__ float s_v[4][16][64];                        // [wave][C element][lane]
    const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, n = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r0 = blockIdx.x * 32, t0 = blockIdx.y * 32;
    const int row = min(r0 + n, A.rows - 1);
    const uint8_t *wr = A.w + (int64_t)row * A.row_stride;
    const int nb = A.K >> 8, rounds = (nb + 3) >> 2;
    constexpr int BB = FMT == F_Q4_K ? 144 : 210;
    // activation pieces of the wave's block: lane -> (token, 16-byte part),
    // 16 lanes per token row, 4 rows per load
    const int8_t *xsrc[8];
    int xdst[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int p = lane + 64 * j, tok = p >> 4, part = p & 15;
        xsrc[j] = A.xq + (int64_t)min(t0 + tok, A.T - 1) * A.K + 16 * part;
        xdst[j] = tok * GEMM_XS + 16 * part;
    }
    int8_t *xs = s_xs[wave];
    int b = min(wave, nb - 1);
    GemmW<FMT> W;
    gemm_w_load(W, wr + (int64_t)b * BB, half);
    {
        uint4 st[8];
#pragma unroll
        for (int j = 0; j < 8; j++) st[j] = *(const uint4 *)(xsrc[j] + 256 * b);
#pragma unroll
        for (int j = 0; j < 8; j++) *(uint4 *)(xs + xdst[j]) = st[j];
    }
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int it = 0; it < rounds; it++) {
        b = 4 * it + wave;
        const bool have = b < nb;
        const int bn = min(b + 4, nb - 1);  // the wave's next block (clamped; unused past the end)
        GemmW<FMT> Wn;
        gemm_w_load(Wn, wr + (int64_t)bn * BB, half);
        float v[16] = {};
        if (have) {
            float4 dv[4];
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++)
                dv[g4] = *(const float4 *)(A.dx + (int64_t)b * A.ldx + t0 + 4 * half + 8 * g4);
            int isum[1][16];
            rh_v16i imin[1];
            gemm_block_ints<1>(W, xs, lane, isum, imin);
            float d, dmin = 0.0f;
            if constexpr (FMT == F_Q4_K) {
                d = h2f(W.hdr.x & 0xFFFF);
                dmin = h2f(W.hdr.x >> 16);
            } else {
                d = h2f(W.d & 0xFFFF);
            }
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const float dxs[4] = {dv[g4].x, dv[g4].y, dv[g4].z, dv[g4].w};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int i = 4 * g4 + r;
                    if constexpr (FMT == F_Q4_K) {
                        const float t1 = d * (float)isum[0][i];
                        const float t2 = dmin * (float)imin[0][i];
                        v[i] = dxs[r] * (t1 - t2);
                    } else {
                        v[i] = (dxs[r] * d) * (float)isum[0][i];
                    }
                }
            }
        }
        // the next block's activations, in flight over the barrier (issued
        // after this block's products, so that they hold no registers there)
        rh_v4i st[8];
#pragma unroll
        for (int j = 0; j < 8; j++) st[j] = *(const rh_v4i *)(xsrc[j] + 256 * bn);
        __syncthreads();  // every wave has read the previous round's values
        if (have) {
#pragma unroll
            for (int i = 0; i < 16; i++) s_v[wave][i][lane] = v[i];
        }
        // (this wave's own tile: its LDS reads above complete before these
        // writes, in program order)
#pragma unroll
        for (int j = 0; j < 8; j++) *(rh_v4i *)(xs + xdst[j]) = st[j];
        __syncthreads();
        // the round's blocks in order, for this wave's four C elements
#pragma unroll
        for (int w2 = 0; w2 < 4; w2++) {
            if (4 * it + w2 >= nb) break;
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] += s_v[w2][4 * wave + e][lane];
        }
        W = Wn;
    }
    if (r0 + n >= A.rows) return;
    const float bias = A.bias ? A.bias[r0 + n] : 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int i = 4 * wave + e;
        const int t = t0 + 8 * (i >> 2) + 4 * half + (i & 3);
        if (t >= A.T) continue;
        float *yp = A.y + (int64_t)t * A.ldy + r0 + n;
        float v = acc[e];
        if (A.bias) v = v + bias;
        if (A.epi == EPI_ADD)
            *yp += v;
        else
            *yp = v;
    }
}

}  // namespace rh
