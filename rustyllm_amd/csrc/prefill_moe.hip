// prefill_moe.hip — batched prefill for the gpt-oss resident decoder.  The
// reference prefills gpt-oss token by token (forward_prefill_gpt_oss,
// src/model.rs:10286, i.e. forward_hidden_gpt_oss_impl without the final
// norm); here a chunk of T prompt tokens goes through each layer together, so
// each dense matrix is read once per token group and each expert matrix once
// per group of the tokens routed to it, while every token's arithmetic is its
// decode step's: the same dot orders, RMSNorm, RoPE, attention, SwiGLU and
// slot-ordered combine.  The kernels here add a token dimension to the decode
// step's kernels; the host side (r_prefill_chunk_moe) strings them together.
#pragma once
#include "attention_exact.hip"
#include "common.hpp"
#include "gemv.hip"
#include "moe.hip"
#include "ops.hip"

namespace rh {

// rms_norm_into of T rows, f32 out: rmsnorm_q8k_kernel's arithmetic per row.
// grid (ceil(n/256), T), dynamic LDS n floats; n % 4 == 0.
__global__ __launch_bounds__(256) void rmsnorm_f32_batch_kernel(const float *x, const float *w, float eps, int n,
                                                                float *xn) {
    const int64_t t = blockIdx.y;
    rmsnorm_row(x + t * n, w, eps, n, xn + t * n, XQ{});
}

// Q8_0 rows for T tokens; each (row, token) is exactly the single-token
// kernel's value: F32, dot_q8_0_f32_avx2 as gemv_q8_0_f32x_kernel (eight
// lane accumulators acc_j = fma(d*q, x[32b + 8i + j], acc_j)); otherwise
// dot_q8_0_q8k_avx2 as gemv_q8_0_pipe_kernel (acc_j = fma(dx*d, s_j, acc_j),
// s_j the exact dot of bytes 4j..4j+3); then hsum_avx, bias, store or add.
// A workgroup is 32 rows (4 waves x 8 rows x 8 lanes, lane j accumulator j)
// by TG tokens whose activations are staged in LDS: F32 float [TG][K]; Q8_K
// int8 [TG][K] then the scales float [TG][K/256].  grid (ceil(rows/32),
// ceil(T/TG)).
struct Q80BatchArgs {
    const uint8_t *w;
    int64_t row_stride;
    int32_t rows, K, T, epi;
    const float *x;    // F32: [T][K]
    const int8_t *qs;  // Q8_K: quants [T][K], scales [K/256][ldx] (token-minor)
    const float *dx;
    int32_t ldx;
    const float *bias;
    float *y;  // [T][ldy]
    int32_t ldy;
};

template <bool F32, int TG>
__global__ __launch_bounds__(256) void gemv_q8_0_batch_kernel(Q80BatchArgs A) {
    extern __shared__ __align__(16) uint8_t s_act[];
    const int K = A.K, nb = K >> 5, tid = threadIdx.x;
    const int t0 = blockIdx.y * TG, tn = min(TG, A.T - t0);
    if (F32) {
        float4 *sx = (float4 *)s_act;
        const int k4 = K / 4;
        for (int i = tid; i < TG * k4; i += 256) {
            const int z = i / k4, c = i - z * k4;
            sx[i] = z < tn ? ((const float4 *)(A.x + (int64_t)(t0 + z) * K))[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    } else {
        int4 *sq = (int4 *)s_act;
        float *sd = (float *)(s_act + (size_t)TG * K);
        const int k16 = K / 16, nsb = K / 256;
        for (int i = tid; i < TG * k16; i += 256) {
            const int z = i / k16, c = i - z * k16;
            sq[i] = z < tn ? ((const int4 *)(A.qs + (int64_t)(t0 + z) * K))[c] : make_int4(0, 0, 0, 0);
        }
        for (int i = tid; i < TG * nsb; i += 256) {
            const int z = i / nsb, b = i - z * nsb;
            sd[i] = z < tn ? A.dx[(int64_t)b * A.ldx + t0 + z] : 0.0f;
        }
    }
    __syncthreads();
    const int lane = tid & 63, wave = tid >> 6, j = lane & 7;
    const int row = blockIdx.x * 32 + wave * 8 + (lane >> 3);
    const bool ok = row < A.rows;
    const uint8_t *rp = A.w + (int64_t)(ok ? row : 0) * A.row_stride;
    float acc[TG];
#pragma unroll
    for (int z = 0; z < TG; z++) acc[z] = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = rp + b * 34;
        const float d = ldh(blk);
        const uint4 q0 = ld16(blk + 2), q1 = ld16(blk + 18);
        if (F32) {
            // byte 8i + j of the 32 quants: dword 2i + j/4, bits 8*(j%4)
            const uint32_t sh = 8u * (uint32_t)(j & 3);
            const bool hi = j >= 4;
            const uint32_t dw[4] = {hi ? q0.y : q0.x, hi ? q0.w : q0.z, hi ? q1.y : q1.x, hi ? q1.w : q1.z};
            float dq[4];
#pragma unroll
            for (int i = 0; i < 4; i++) dq[i] = d * (float)(int)__builtin_amdgcn_sbfe((int)dw[i], sh, 8u);
            const float *sx = (const float *)s_act + b * 32 + j;
#pragma unroll
            for (int z = 0; z < TG; z++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[z] = fmaf(dq[i], sx[(size_t)z * K + 8 * i], acc[z]);
        } else {
            const uint32_t wsel[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            uint32_t wj = wsel[0];
#pragma unroll
            for (int i = 1; i < 8; i++) wj = j == i ? wsel[i] : wj;
            const int32_t *sq = (const int32_t *)s_act;
            const float *sd = (const float *)(s_act + (size_t)TG * K);
#pragma unroll
            for (int z = 0; z < TG; z++) {
                const float sc = sd[z * (K / 256) + (b >> 3)] * d;
                const int s = sdot4(wj, sq[(size_t)z * (K / 4) + b * 8 + j], 0);
                acc[z] = fmaf(sc, (float)s, acc[z]);
            }
        }
    }
#pragma unroll
    for (int z = 0; z < TG; z++) {
        // hsum_avx: t_i = a_i + a_{i+4}; ((t0+t1) + (t2+t3))
        const float t = acc[z] + __shfl_xor(acc[z], 4, 64);
        const float u = t + __shfl_xor(t, 1, 64);
        float v = u + __shfl_xor(u, 2, 64);
        if (z < tn && ok && j == 0) {
            if (A.bias) v += A.bias[row];
            float *y = A.y + (int64_t)(t0 + z) * A.ldy + row;
            if (A.epi == EPI_ADD)
                *y += v;
            else
                *y = v;
        }
    }
}

// Router selection of T tokens (moe_topk_kernel per token): logits [T][ldl],
// sel / prob [T][k].  grid T.
__global__ __launch_bounds__(64) void moe_topk_batch_kernel(const float *logits, int ldl, int n, int k, int32_t *sel,
                                                            float *prob) {
    const int64_t t = blockIdx.x;
    moe_topk_row(logits + t * ldl, n, k, sel + t * k, prob + t * k);
}

// x[t] += sum over slots r in order of (proj[t k + r] + db[e_r]) * p_r, per
// token (moe_combine_kernel).  grid (ceil(dim/256), T).
__global__ __launch_bounds__(256) void moe_combine_batch_kernel(const float *proj, int dim, int k, const int32_t *sel,
                                                                const float *prob, const float *db, int db_stride,
                                                                float *x) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int64_t t = blockIdx.y;
    if (i >= dim) return;
    float acc = 0.0f;
    for (int r = 0; r < k; r++) {
        const int64_t p = t * k + r;
        float v = proj[p * dim + i];
        if (db) v = v + db[(size_t)sel[p] * db_stride + i];
        acc += v * prob[p];
    }
    x[t * dim + i] += acc;
}

// MXFP4 expert rows for the (token, slot) pairs routed to each expert, every
// sum dot_mxfp4_f32_scalar's running sum (as the single-token kernels).  A
// workgroup of four waves serves one (64-row tile, expert, matrix): it lists
// the pairs p = t k + r with sel[p] == expert, then in passes of 4 x MXE_G
// pairs (wave w takes MXE_G of them, one running sum per pair and lane = row)
// streams the tile's rows once per pass in 16-block chunks: coalesced direct
// loads into a double-buffered LDS chunk (64 rows x 272 bytes, 17 loads of 1
// KB shared among the waves), from which every lane reads its row's 17-byte
// blocks.  A block's 32 weights are decoded once per wave and used for all
// of its pairs; x comes through scalar loads.  y[mat] row p gets pair p's
// sum.  grid (ceil(rows/64), n_exp, n_mats).
#define MXE_G 8
#define MXE_MAX_PAIRS 1024  // a token routes to an expert at most once: pairs per expert <= T
struct MxExpArgs {
    const uint8_t *w[2];  // expert tensors: expert e's row r at w + e*exp_stride + r*row_stride
    float *y[2];          // [T*k][ldy]
    int64_t row_stride, exp_stride;
    int32_t rows, K, n_pairs, k;
    const float *x;  // the activation of pair p: x + (x_pair ? p : p / k) * ldx
    int64_t ldx, ldy;
    int32_t x_pair;
    const int32_t *sel;  // [n_pairs]
    int32_t n_exp;       // the matrix-core kernel's expert count
};

__global__ __launch_bounds__(256) void gemv_mxfp4_experts_kernel(MxExpArgs A) {
    __shared__ __align__(16) uint4 s_b[2][64 * 17];
    __shared__ int32_t s_list[MXE_MAX_PAIRS];
    __shared__ int32_t s_cnt[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int e = blockIdx.y, mat = blockIdx.z;
    const int K = A.K, nb = K >> 5;
    // the pairs routed to expert e, in pair order: each wave counts a quarter
    // of the pairs, then writes its hits after the earlier waves'
    const int per = (A.n_pairs + 3) / 4, pa = wave * per, pb = min(A.n_pairs, pa + per);
    int cnt = 0;
    for (int base = pa; base < pb; base += 64) {
        const int p = base + lane;
        cnt += __builtin_popcountll(__builtin_amdgcn_ballot_w64(p < pb && A.sel[p] == e));
    }
    if (lane == 0) s_cnt[wave] = cnt;
    __syncthreads();
    int off = 0, n = 0;
    for (int i = 0; i < 4; i++) {
        off += i < wave ? s_cnt[i] : 0;
        n += s_cnt[i];
    }
    for (int base = pa; base < pb; base += 64) {
        const int p = base + lane;
        const bool hit = p < pb && A.sel[p] == e;
        const unsigned long long m = __builtin_amdgcn_ballot_w64(hit);
        const int at = off + __builtin_popcountll(m & ((1ull << lane) - 1ull));
        if (hit && at < MXE_MAX_PAIRS) s_list[at] = p;
        off += __builtin_popcountll(m);
    }
    // the callers route every token to an expert at most once, so n <= T <=
    // MXE_MAX_PAIRS; the bound only keeps the list inside its array
    n = min(n, MXE_MAX_PAIRS);
    if (n == 0) return;  // uniform over the workgroup
    __syncthreads();
    const uint8_t *w = A.w[mat] + (int64_t)e * A.exp_stride;
    const int row0 = blockIdx.x * 64, row = row0 + lane;
    const bool live = row < A.rows;
    const int64_t stride = A.row_stride;
    const int nch = (nb + MXF_C - 1) / MXF_C;
    // piece f = 64 i + lane of a chunk is row f / 17, bytes 16 (f % 17); wave
    // w issues pieces i = w, w + 4, ...
    auto issue_chunk = [&](int c, int buf) {
        for (int i = wave; i < 17; i += 4) {
            const int f = 64 * i + lane, r = f / 17, p = f - 17 * r;
            const int rr = min(row0 + r, A.rows - 1);
            const int64_t o = min((int64_t)(MXF_C * 17 * c + 16 * p), stride - 16);
            dma16(w + (int64_t)rr * stride + o, &s_b[buf][64 * i]);
        }
    };
    for (int g0 = 0; g0 < n; g0 += 4 * MXE_G) {
        const int q0 = g0 + wave * MXE_G;  // this wave's first pair of the pass
        const float *xp[MXE_G];
#pragma unroll
        for (int i = 0; i < MXE_G; i++) {
            // uniform, so that x arrives through scalar loads
            const int p = __builtin_amdgcn_readfirstlane(s_list[min(q0 + i, n - 1)]);
            xp[i] = A.x + (A.x_pair ? (int64_t)p : (int64_t)(p / A.k)) * A.ldx;
        }
        float sum[MXE_G];
#pragma unroll
        for (int i = 0; i < MXE_G; i++) sum[i] = 0.0f;
        issue_chunk(0, 0);
        for (int c = 0; c < nch; c++) {
            RH_WAIT_VM(0);
            __syncthreads();  // chunk c landed from every wave; chunk c - 1's reads are done
            if (c + 1 < nch) issue_chunk(c + 1, (c + 1) & 1);
            const uint8_t *rowb = (const uint8_t *)&s_b[c & 1][17 * lane];
            for (int jj = 0; jj < MXF_C / 4; jj++) {
#pragma unroll
            for (int o = 0; o < 4; o++) {
                const int j = 4 * jj + o, b = MXF_C * c + j;
                if (b >= nb) break;  // uniform
                // block j's 17 bytes start at byte 17 j = 68 jj + 16 o + o of
                // the row: five dwords from the aligned 68 jj + 16 o, shifted
                // by o bytes
                const uint32_t *wp = (const uint32_t *)(rowb + 68 * jj + 16 * o);
                uint32_t dw[5];
#pragma unroll
                for (int i = 0; i < 5; i++) dw[i] = wp[i];
                uint32_t wd[4];
#pragma unroll
                for (int k4 = 0; k4 < 4; k4++) wd[k4] = o ? __builtin_amdgcn_alignbyte(dw[k4 + 1], dw[k4], o) : dw[k4];
                const uint32_t e4 = dw[4] >> (8 * o);
                const uint32_t ex = e4 & 0xFFu;
                const float sc = mxfp4_scale(ex);
                // the block's 32 weights lut * scale, exact either way
                float wv[32];
                if (__builtin_amdgcn_ballot_w64(ex == 0u || ex == 255u) == 0) {
#pragma unroll
                    for (int k4 = 0; k4 < 4; k4++)
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            const fp4x2_f32 pr = fp4x2_scaled(wd[k4], sc, u);
                            wv[8 * k4 + 2 * u] = pr.x;
                            wv[8 * k4 + 2 * u + 1] = pr.y;
                        }
                } else {
#pragma unroll
                    for (int k4 = 0; k4 < 4; k4++)
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            const uint32_t byte = (wd[k4] >> (8 * u)) & 0xFFu;
                            wv[8 * k4 + 2 * u] = mxfp4_nibble(byte & 0xFu) * sc;
                            wv[8 * k4 + 2 * u + 1] = mxfp4_nibble(byte >> 4) * sc;
                        }
                }
#pragma unroll
                for (int i = 0; i < MXE_G; i++) {
                    const const_f32_ptr xb = (const_f32_ptr)xp[i] + b * 32;
#pragma unroll
                    for (int q = 0; q < 32; q++) sum[i] += wv[q] * xb[q];
                }
            }
            }
        }
        __syncthreads();  // the last chunk's reads are done before the next pass restages
#pragma unroll
        for (int i = 0; i < MXE_G; i++)
            if (q0 + i < n && live) A.y[mat][(int64_t)s_list[q0 + i] * A.ldy + row] = sum[i];
    }
}

// ---- opt-in expert product on the matrix cores ------------------------------
// The reference sums each MXFP4 row serially (dot_mxfp4_f32_scalar); the
// matrix cores sum in their own order, so this path is not bit-exact and is
// off unless rusty_hip_set_expert_mfma(1) selects it.  Its inputs keep the
// reference's precision: the weights lut[n] * 2^(e-127) are exact in f32 and
// the activations are the f32 rows; only the order of the f32 additions of
// the K products differs (v_mfma_f32_32x32x2_f32).
//
// moe_expert_lists_kernel: for every expert, the pairs routed to it in pair
// order (lists[e * cap ..]), their count, and tile0[e] = the number of
// 32-pair tiles of the experts before e (tile0[n_exp] = all tiles).  One
// workgroup; wave w lists experts w, w + 4, ...
#define MXM_PAIRS 32
#define MXM_ROWS 128
__global__ __launch_bounds__(256) void moe_expert_lists_kernel(const int32_t *sel, int n_pairs, int n_exp, int cap,
                                                               int32_t *lists, int32_t *counts, int32_t *tile0) {
    __shared__ int32_t s_cnt[64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int e = wave; e < n_exp; e += 4) {
        int cnt = 0;
        for (int base = 0; base < n_pairs; base += 64) {
            const int p = base + lane;
            const bool hit = p < n_pairs && sel[p] == e;
            const unsigned long long m = __builtin_amdgcn_ballot_w64(hit);
            const int at = cnt + __builtin_popcountll(m & ((1ull << lane) - 1ull));
            if (hit && at < cap) lists[(size_t)e * cap + at] = p;
            cnt += __builtin_popcountll(m);
        }
        cnt = min(cnt, cap);
        if (lane == 0) {
            counts[e] = cnt;
            s_cnt[e] = cnt;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int t = 0;
        for (int e = 0; e < n_exp; e++) {
            tile0[e] = t;
            t += (s_cnt[e] + MXM_PAIRS - 1) / MXM_PAIRS;
        }
        tile0[n_exp] = t;
    }
}

// y[mat] row p = expert rows times pair p's activation for one (128-row tile,
// 32-pair tile of one expert, matrix): grid (ceil(rows / 128), an upper bound
// of the pair tiles, n_mats); workgroups past tile0[n_exp] return.  Wave w
// owns rows row0 + 32 w + (lane % 32); per 32-element block, 16 MFMAs
// 32x32x2: MFMA i takes element 16 h + i (h = lane / 32) of the block from
// both operands, A = the pair's activation (m = pair), B = the weight (n =
// row), so lane h decodes bytes 8h..8h+7 of its row's block (element 2b + 1
// is the high nibble of byte b).  The weights arrive in 16-block chunks of
// 272 bytes per row by coalesced direct loads into a double-buffered LDS
// chunk; each lane then reads its row's chunk into registers (17 reads, an
// odd number of 16-byte units per row: conflict-free); the activations come
// from global memory one block ahead.
__global__ __launch_bounds__(256) void gemm_mxfp4_experts_mfma_kernel(MxExpArgs A, const int32_t *lists,
                                                                      const int32_t *counts, const int32_t *tile0,
                                                                      int cap) {
    __shared__ __align__(16) uint4 s_b[2][MXM_ROWS * 17];
    __shared__ int32_t s_pair[MXM_PAIRS];
    typedef float v16f __attribute__((ext_vector_type(16)));
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int mat = blockIdx.z, gt = blockIdx.y;
    const int n_exp = A.n_exp;
    if (gt >= tile0[n_exp]) return;  // uniform
    int e = 0;
    while (e + 1 < n_exp && tile0[e + 1] <= gt) e++;
    const int p0 = (gt - tile0[e]) * MXM_PAIRS;
    const int np = min(MXM_PAIRS, counts[e] - p0);
    if (tid < MXM_PAIRS) s_pair[tid] = lists[(size_t)e * cap + p0 + min(tid, np - 1)];
    const int m = lane & 31, h = lane >> 5;
    const int row0 = blockIdx.x * MXM_ROWS, row = row0 + 32 * wave + m;
    const uint8_t *w = A.w[mat] + (int64_t)e * A.exp_stride;
    const int64_t stride = A.row_stride;
    const int nb = A.K >> 5, nch = (nb + MXF_C - 1) / MXF_C;
    // piece f = 256 i + tid of a chunk: row f / 17, bytes 16 (f % 17); the
    // 2176 pieces are 34 whole wave instructions, so a wave's instruction is
    // either all inside the chunk or skipped
    auto issue_chunk = [&](int c, int buf) {
#pragma unroll
        for (int i = 0; i < 9; i++) {
            if (256 * i + 64 * wave >= MXM_ROWS * 17) continue;  // uniform
            const int f = 256 * i + tid, r = f / 17, pc = f - 17 * r;
            const int rr = min(row0 + r, A.rows - 1);
            const int64_t o = min((int64_t)(MXF_C * 17 * c + 16 * pc), stride - 16);
            dma16(w + (int64_t)rr * stride + o, &s_b[buf][256 * i + 64 * wave]);
        }
    };
    issue_chunk(0, 0);
    __syncthreads();  // s_pair
    const int pair = s_pair[m];
    const float *xr = A.x + (A.x_pair ? (int64_t)pair : (int64_t)(pair / A.k)) * A.ldx + 16 * h;
    float4 xa[4], xb[4];
    auto load_x = [&](int b, float4 (&xv)[4]) {
        const float4 *p = (const float4 *)(xr + 32 * (int64_t)min(b, nb - 1));
#pragma unroll
        for (int q = 0; q < 4; q++) xv[q] = p[q];
    };
    load_x(0, xa);
    v16f acc = {};
    for (int c = 0; c < nch; c++) {
        RH_WAIT_VM(0);
        __syncthreads();  // chunk c landed from every wave; every read of chunk c - 1 done
        uint32_t wr[68];
        {
            const uint4 *rp = &s_b[c & 1][(32 * wave + m) * 17];
#pragma unroll
            for (int q = 0; q < 17; q++) {
                const uint4 v = rp[q];
                wr[4 * q] = v.x;
                wr[4 * q + 1] = v.y;
                wr[4 * q + 2] = v.z;
                wr[4 * q + 3] = v.w;
            }
        }
        // block j of the chunk with its activations in cur; the next block's
        // go to nxt (clamped past the end), then, late in the chunk, the next
        // chunk's weights are issued: a load issued after them would wait for
        // them too (loads retire in order), and only the next chunk's first
        // activations are
        auto block = [&](int j, const float4 (&cur)[4], float4 (&nxt)[4]) {
            const int b = MXF_C * c + j;
            if (b >= nb) return;  // uniform
            load_x(b + 1, nxt);
            if (j == MXF_C - 2 && c + 1 < nch) issue_chunk(c + 1, (c + 1) & 1);
            // bytes 17 j + 8 h .. + 7 and the scale byte 17 j + 16
            const int o0 = 17 * j, o1 = 17 * j + 8, os = 17 * j + 16;
            const uint32_t a0 = __builtin_amdgcn_alignbyte(wr[o0 / 4 + 1], wr[o0 / 4], o0 % 4);
            const uint32_t a1 = __builtin_amdgcn_alignbyte(wr[o0 / 4 + 2], wr[o0 / 4 + 1], o0 % 4);
            const uint32_t c0 = __builtin_amdgcn_alignbyte(wr[o1 / 4 + 1], wr[o1 / 4], o1 % 4);
            const uint32_t c1 = __builtin_amdgcn_alignbyte(wr[o1 / 4 + 2], wr[o1 / 4 + 1], o1 % 4);
            const uint32_t d0 = h ? c0 : a0, d1 = h ? c1 : a1;
            const uint32_t ex = (wr[os / 4] >> (8 * (os % 4))) & 0xFFu;
            const float sc = mxfp4_scale(ex);
            float wv[16];
            if (__builtin_amdgcn_ballot_w64(ex == 0u || ex == 255u) == 0) {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const fp4x2_f32 lo = fp4x2_scaled(d0, sc, u), hi = fp4x2_scaled(d1, sc, u);
                    wv[2 * u] = lo.x;
                    wv[2 * u + 1] = lo.y;
                    wv[8 + 2 * u] = hi.x;
                    wv[9 + 2 * u] = hi.y;
                }
            } else {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const uint32_t b0 = (d0 >> (8 * u)) & 0xFFu, b1 = (d1 >> (8 * u)) & 0xFFu;
                    wv[2 * u] = mxfp4_nibble(b0 & 0xFu) * sc;
                    wv[2 * u + 1] = mxfp4_nibble(b0 >> 4) * sc;
                    wv[8 + 2 * u] = mxfp4_nibble(b1 & 0xFu) * sc;
                    wv[9 + 2 * u] = mxfp4_nibble(b1 >> 4) * sc;
                }
            }
            const float xs[16] = {cur[0].x, cur[0].y, cur[0].z, cur[0].w, cur[1].x, cur[1].y, cur[1].z, cur[1].w,
                                  cur[2].x, cur[2].y, cur[2].z, cur[2].w, cur[3].x, cur[3].y, cur[3].z, cur[3].w};
#pragma unroll
            for (int i = 0; i < 16; i++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xs[i], wv[i], acc, 0, 0, 0);
        };
#pragma unroll
        for (int j = 0; j < MXF_C; j += 2) {
            block(j, xa, xb);
            block(j + 1, xb, xa);
        }
    }
    if (row >= A.rows) return;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int mi = 8 * (i >> 2) + 4 * h + (i & 3);
        if (mi < np) A.y[mat][(int64_t)s_pair[mi] * A.ldy + row] = acc[i];
    }
}

// K/V rows between a ring cache and the linear buffer of a batched ring
// prefill: gather lin[r] = ring[(p0 + r) % S] for r < n rows; scatter
// ring[(p0 + r) % S] = lin[off + r].  grid (ceil(width/256), n, 2 (K, V)).
__global__ __launch_bounds__(256) void kv_ring_copy_kernel(float *kring, float *vring, float *klin, float *vlin,
                                                           int kw, int vw, int p0, int S, int off, int to_ring) {
    const int r = blockIdx.y, which = blockIdx.z, c = blockIdx.x * 256 + threadIdx.x;
    const int w = which ? vw : kw;
    if (c >= w) return;
    float *ring = which ? vring : kring;
    float *lin = which ? vlin : klin;
    const int64_t slot = (p0 + r) % S;
    if (to_ring)
        ring[slot * w + c] = lin[(int64_t)(off + r) * w + c];
    else
        lin[(int64_t)r * w + c] = ring[slot * w + c];
}

}  // namespace rh
