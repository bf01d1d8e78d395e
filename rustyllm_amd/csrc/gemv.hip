// gemv.hip — fused dequant-dot matrix-vector kernels for gfx950 (wave64).
//
// Weights stay in raw GGUF block bytes (device copy of the tensor, rows padded
// to a 16-byte stride).  Activations arrive already quantized to Q8_K (int8 per
// element, f32 scale per 256, int16 sums per 32 and per 16) for Q4_K, Q6_K and
// Q8_0 with K % 256 == 0, exactly as the reference's x86 path does
// (prepare_xq_kquant, src/simd.rs:944-959); Q8_0 with other K and MXFP4 read
// f32 activations (src/simd.rs:6671-6692, 5886-5902).
//
// Work split: a 256-thread workgroup owns a tile of 4*R consecutive rows, R per
// wave.  Inside a wave, lane l handles "unit" l + 64*i of the row (i <
// ITERS): a quarter of a 256-block for K-quants (64 weights), one whole
// 32-block for Q8_0/MXFP4.  Integer partial sums are exact, so their lane
// order is free; each block's f32 value is then formed with the reference's
// own rounding sequence and the per-row sum runs serially in block order, so
// Q4_K, Q6_K and Q8_0 (int) rows reproduce the reference row bit for bit.
#pragma once
#include "common.hpp"

#include <type_traits>

namespace rh {

enum Fmt : int { F_Q8_0 = 8, F_Q4_K = 12, F_Q6_K = 14, F_MXFP4 = 39 };

// Epilogue of a matrix inside a launch.
enum Epi : int {
    EPI_STORE = 0,   // y[r] = v (+ bias)
    EPI_ADD = 1,     // y[r] += v (+ bias): residual stream update
    EPI_SWIGLU = 2,  // matrices 0 (gate) and 1 (up): y[r] = silu(g) * u
};

struct GemvMat {
    const uint8_t *w;
    int64_t row_stride;  // bytes between device rows (>= raw row bytes, 16-aligned)
    int32_t rows;
    int32_t fmt;
    float *y;
    const float *bias;
    int32_t tile_begin;  // first tile index of this matrix in the launch
    int32_t sel_b;       // with sel: floats between the experts' bias rows
    const float *x;      // f32-activation kernels: this matrix's activation (null: the launch's)
    const int32_t *sel;  // expert chosen on the device: w += *sel * sel_w, bias += *sel * sel_b
    int64_t sel_w;       // with sel: bytes between the experts' matrices
};

#define GEMV_MAX_MATS 8

// Where a K-quant launch's Q8_K activation comes from.  KQ_ACT_XQ: a Q8_K
// vector in memory (xq).  The others build it in every workgroup's prologue,
// from f32 data, while the first tiles' weights are in flight, which saves
// the standalone kernel (and its launch) that would otherwise produce it:
//   KQ_ACT_NORM: RMSNorm of act_x with act_w (rms_norm_into), then Q8_K;
//   KQ_ACT_DEN:  attention normalisation act_x[e] * (1/act_den[e/act_group])
//                where the denominator is positive, then Q8_K;
//   KQ_ACT_QUANT: Q8_K of act_x as is (quantize_row_q8k), up to four chunks
//                per thread.
//   KQ_ACT_NORM2 / KQ_ACT_DEN2: the same for 4096 < K < 8192, two 16-element
//                chunks per thread.
enum KqAct : int { KQ_ACT_XQ = 0, KQ_ACT_NORM = 1, KQ_ACT_DEN = 2, KQ_ACT_QUANT = 3, KQ_ACT_NORM2 = 4, KQ_ACT_DEN2 = 5 };
#define KQ_ACT_KMAX 4096        // widest activation NORM / DEN build: one 16-element chunk per thread
#define KQ_ACT_KMAX2 8191       // NORM2 / DEN2: two chunks per thread (rows of fewer than 32 blocks)
#define KQ_ACT_QUANT_KMAX 16384  // QUANT: four chunks per thread

struct GemvArgs {
    GemvMat m[GEMV_MAX_MATS];
    int32_t n_mats;
    int32_t n_tiles;
    int32_t K;
    int32_t epi;
    int32_t tile_rows;  // K-quant kernel: rows per wave tile (per matrix for SWIGLU)
    XQ xq;              // Q8_K activation (int paths)
    const float *x;     // f32 activation (f32 paths)
    // K-quant prologue activation (KqAct != KQ_ACT_XQ)
    const float *act_x;
    const float *act_w;
    const float *act_den;
    float act_eps;
    int32_t act_group;
    int32_t act_store;  // prologue modes: workgroup 0 also writes the Q8_K vector it built to xq
    // MoE expert launches (MXFP4 one-wave kernel): the router's topk_n logits
    // are ranked in every workgroup (moe_topk_row's selection) and slot r =
    // GemvMat::sel - topk_sel takes the rank-r expert instead of reading
    // *sel; workgroup 0 also stores every slot's expert and weight to
    // topk_sel / topk_prob for the later launches.  null: *sel as given.
    const float *topk_logits;
    int32_t topk_n, topk_k;
    int32_t *topk_sel;
    float *topk_prob;
    // Q8_0 f32-activation kernel, NORM instance: the staged activation is
    // replaced by its RMSNorm with norm_w (rms_norm_into's sum order and expression), and
    // workgroup 0 also stores the normalised vector to norm_out.
    const float *norm_w;
    float norm_eps;
    float *norm_out;
};
// byte offset of a kernel's second GemvArgs argument in its argument segment
constexpr int KARG_SECOND = (int)((sizeof(GemvArgs) + alignof(GemvArgs) - 1) / alignof(GemvArgs) * alignof(GemvArgs));

// Matrix mi of a launch with mi wave-uniform.  The byval kernel argument
// must not be indexed with a run-time value (the compiler then copies it to
// scratch and reads it back with vector loads followed by vmcnt(0) waits,
// which drain every weight load in flight).  The descriptor is read instead
// through the kernarg segment pointer, at the argument's offset KOFF (0 for
// a kernel's first argument), so these are scalar loads at a uniform offset.
typedef const __attribute__((address_space(4))) GemvArgs KGemvArgs;
template <int KOFF = 0>
__device__ __forceinline__ GemvMat mat_sel(const GemvArgs &, int mi) {
    KGemvArgs *ka =
        (KGemvArgs *)((const __attribute__((address_space(4))) char *)__builtin_amdgcn_kernarg_segment_ptr() + KOFF);
    GemvMat r;
    r.w = ka->m[mi].w;
    r.row_stride = ka->m[mi].row_stride;
    r.rows = ka->m[mi].rows;
    r.fmt = ka->m[mi].fmt;
    r.y = ka->m[mi].y;
    r.bias = ka->m[mi].bias;
    r.tile_begin = ka->m[mi].tile_begin;
    r.sel_b = ka->m[mi].sel_b;
    r.x = ka->m[mi].x;
    r.sel = ka->m[mi].sel;
    r.sel_w = ka->m[mi].sel_w;
    return r;
}

#define KMAX 16384
#define NB256_MAX (KMAX / 256)
#define NB32_MAX (KMAX / 32)

// Cephes-style expf restated from the reference's silu_mul_avx2
// (src/simd.rs:2406-2464, constants :2410-2421), step for step, so SiLU on the
// GPU rounds exactly like the AVX2 path.
__device__ __forceinline__ float exp_cephes(float x) {
    x = fminf(88.37626f, fmaxf(-88.37626f, x));
    float fx = fmaf(x, 1.44269504088896340736f, 0.5f);
    fx = floorf(fx);
    x = fmaf(-fx, 0.6933594f, x);
    x = fmaf(-fx, -2.1219444e-4f, x);
    float y = 1.9875691e-4f;
    y = fmaf(y, x, 1.3982e-3f);
    y = fmaf(y, x, 8.333452e-3f);
    y = fmaf(y, x, 4.1665796e-2f);
    y = fmaf(y, x, 1.6666665e-1f);
    y = fmaf(y, x, 0.5f);
    float x2 = x * x;
    y = fmaf(y, x2, x) + 1.0f;
    int n = (int)fx;
    float p2 = __builtin_bit_cast(float, (n + 0x7f) << 23);
    return y * p2;
}

__device__ __forceinline__ float silu_mul_ref(float g, float u) {
    float e = exp_cephes(0.0f - g);
    float s = g / (1.0f + e);
    return s * u;
}

// get_scale_min_k4 (src/simd.rs:4537-4546) on the 12 scale bytes held in
// three dwords (s03 = bytes 0..3, s47 = 4..7, s811 = 8..11).
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s03, uint32_t s47, uint32_t s811, int &sc, int &m) {
    if (j < 4) {
        sc = (s03 >> (8 * j)) & 63;
        m = (s47 >> (8 * j)) & 63;
    } else {
        int k = j - 4;
        uint32_t a = (s811 >> (8 * k)) & 0xFF;
        sc = (a & 0xF) | (((s03 >> (8 * k + 6)) & 3) << 4);
        m = (a >> 4) | (((s47 >> (8 * k + 6)) & 3) << 4);
    }
}

// ---- K-quant units ----------------------------------------------------------
// Q4_K unit q of block b: 32 qs bytes (offset 16+32q) = 64 weights; low
// nibbles pair with xq[64q .. 64q+32), high nibbles with xq[64q+32 .. 64q+64).
struct Q4KLoad {
    uint4 hdr, a, b;
};
__device__ __forceinline__ Q4KLoad q4k_load(const uint8_t *blk, int q) {
    Q4KLoad L;
    L.hdr = *(const uint4 *)blk;  // 144-byte blocks of 16-aligned rows are 16-aligned
    L.a = *(const uint4 *)(blk + 16 + 32 * q);
    L.b = *(const uint4 *)(blk + 32 + 32 * q);
    return L;
}

// Scale/min fields of quarter q (sub-blocks 2q and 2q+1) in get_scale_min_k4
// (src/simd.rs:4537-4546): sub-block j < 4 is 6 bits of byte j of words 0
// (scale) and 1 (min); j >= 4 is 4 bits of byte j-4 of word 2 with the top 2
// bits of byte j-4 of word 0 / 1 above them.  q is fixed per lane, so both
// forms become one bit-field extract of a selected word plus a second
// extract (zero width for j < 4) shifted in at bit 4, with no branch.
struct Q4KScaleSel {
    bool hi;  // q >= 2
    uint32_t sh_sc[2], sh_m[2], sh_hb[2], w_lo, w_hb;
};
__device__ __forceinline__ Q4KScaleSel q4k_scale_sel(int q) {
    Q4KScaleSel S;
    S.hi = q >= 2;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int j = 2 * q + t, k = j - 4;
        S.sh_sc[t] = S.hi ? 8 * k : 8 * j;
        S.sh_m[t] = S.hi ? 8 * k + 4 : 8 * j;
        S.sh_hb[t] = S.hi ? 8 * k + 6 : 0;
    }
    S.w_lo = S.hi ? 4 : 6;
    S.w_hb = S.hi ? 2 : 0;
    return S;
}
__device__ __forceinline__ void q4k_scale_min(const Q4KScaleSel &S, int t, uint32_t s03, uint32_t s47, uint32_t s811,
                                              int &sc, int &m) {
    const uint32_t a_sc = S.hi ? s811 : s03, a_m = S.hi ? s811 : s47;
    sc = (int)(__builtin_amdgcn_ubfe(a_sc, S.sh_sc[t], S.w_lo) | (__builtin_amdgcn_ubfe(s03, S.sh_hb[t], S.w_hb) << 4));
    m = (int)(__builtin_amdgcn_ubfe(a_m, S.sh_m[t], S.w_lo) | (__builtin_amdgcn_ubfe(s47, S.sh_hb[t], S.w_hb) << 4));
}

// Returns the exact partial (isum, imin) of this quarter.
__device__ __forceinline__ void q4k_unit(const Q4KLoad &L, int q, const Q4KScaleSel &S, const int32_t *xq32,
                                         const int16_t *bs, int &isum, int &imin) {
    int sc1, m1, sc2, m2;
    q4k_scale_min(S, 0, L.hdr.y, L.hdr.z, L.hdr.w, sc1, m1);
    q4k_scale_min(S, 1, L.hdr.y, L.hdr.z, L.hdr.w, sc2, m2);
    const uint32_t w[8] = {L.a.x, L.a.y, L.a.z, L.a.w, L.b.x, L.b.y, L.b.z, L.b.w};
    const int4 *xl = (const int4 *)(xq32 + 16 * q);
    int4 x0 = xl[0], x1 = xl[1], x2 = xl[2], x3 = xl[3];
    const int xv[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w,
                        x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
    int slo0 = 0, slo1 = 0, shi0 = 0, shi1 = 0;  // four short chains instead of two long ones
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
        slo0 = sdot4(w[k] & 0x0F0F0F0Fu, (uint32_t)xv[k], slo0);
        shi0 = sdot4((w[k] >> 4) & 0x0F0F0F0Fu, (uint32_t)xv[8 + k], shi0);
        slo1 = sdot4(w[k + 1] & 0x0F0F0F0Fu, (uint32_t)xv[k + 1], slo1);
        shi1 = sdot4((w[k + 1] >> 4) & 0x0F0F0F0Fu, (uint32_t)xv[9 + k], shi1);
    }
    const int slo = slo0 + slo1, shi = shi0 + shi1;
    const int bsw = *(const int *)(bs + 2 * q);  // bsums of sub-blocks 2q, 2q+1
    // 24-bit products are exact here (|slo|, |shi| <= 32*15*128, scales and
    // mins < 64, |bsums| <= 32*128) and issue at full rate.
    isum = __mul24(sc2, shi) + __mul24(sc1, slo);
    imin = __mul24(m2, bsw >> 16) + __mul24(m1, (int)(int16_t)(bsw & 0xFFFF));
}

// Q6_K unit q = (g = q>>1, j = q&1) of block b: positions l in [16j, 16j+16) of
// half g, i.e. elements 128g + 32k + l for k = 0..3 (64 weights).
struct Q6KLoad {
    uint4 ql0, ql1, qh;
    uint2 sc;
    uint32_t d;
};
__device__ __forceinline__ Q6KLoad q6k_load(const uint8_t *blk, int q) {
    int g = q >> 1, j = q & 1;
    Q6KLoad L;
    L.ql0 = ld16(blk + 64 * g + 16 * j);
    L.ql1 = ld16(blk + 64 * g + 32 + 16 * j);
    L.qh = ld16(blk + 128 + 32 * g + 16 * j);
    L.sc = ld8(blk + 192 + 8 * g);
    L.d = ld2(blk + 208);
    return L;
}

__device__ __forceinline__ int q6k_unit(const Q6KLoad &L, int q, const int32_t *xqb32, const int16_t *s16b) {
    int g = q >> 1, j = q & 1;
    const uint32_t l0[4] = {L.ql0.x, L.ql0.y, L.ql0.z, L.ql0.w};
    const uint32_t l1[4] = {L.ql1.x, L.ql1.y, L.ql1.z, L.ql1.w};
    const uint32_t h[4] = {L.qh.x, L.qh.y, L.qh.z, L.qh.w};
    int isum = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int e0 = 128 * g + 32 * k + 16 * j;  // first element of this 16-run
        const int4 *xp = (const int4 *)(xqb32 + e0 / 4);
        int4 xv = xp[0];
        const int xa[4] = {xv.x, xv.y, xv.z, xv.w};
        int dot = 0;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            uint32_t lo = (k & 1) ? l1[t] : l0[t];
            uint32_t nib = (k & 2) ? ((lo >> 4) & 0x0F0F0F0Fu) : (lo & 0x0F0F0F0Fu);
            uint32_t hb = ((h[t] >> (2 * k)) & 0x03030303u) << 4;
            dot = sdot4(nib | hb, (uint32_t)xa[t], dot);
        }
        dot -= 32 * (int)s16b[e0 / 16];
        int sidx = j + 2 * k;  // scale byte sc[8g + j + 2k]
        uint32_t sw = sidx < 4 ? L.sc.x : L.sc.y;
        int sc = (int)(int8_t)((sw >> (8 * (sidx & 3))) & 0xFF);
        isum += __mul24(sc, dot);  // |dot| <= 16*64*128: exact in 24 bits
    }
    return isum;
}

// One unit's raw bytes: Q4_K uses a = header (d, dmin, 12 scale bytes),
// b/c = its 32 qs bytes; Q6_K uses a/b = ql bytes, c = qh bytes, sc = its 8
// scale bytes, dd = d.
struct UnitLoad {
    uint4 a, b, c;
    uint2 sc;
    uint32_t dd;
};

template <int FMT>
__device__ __forceinline__ void unit_load(const uint8_t *blk, int q, UnitLoad &L) {
    if (FMT == F_Q4_K) {
        L.a = *(const uint4 *)blk;  // 144-byte blocks of 16-aligned rows are 16-aligned
        L.b = *(const uint4 *)(blk + 16 + 32 * q);
        L.c = *(const uint4 *)(blk + 32 + 32 * q);
    } else {
        int g = q >> 1, j = q & 1;
        L.a = ld16(blk + 64 * g + 16 * j);
        L.b = ld16(blk + 64 * g + 32 + 16 * j);
        L.c = ld16(blk + 128 + 32 * g + 16 * j);
        L.sc = ld8(blk + 192 + 8 * g);
        L.dd = ld2(blk + 208);
    }
}

// f32 value of one 256-block from its four units (one per lane of a quad).
// The integer parts are exact; the f32 combine is the reference's own
// sequence (dot_q4_k_q8k_avx2: dx*(d*isum - dmin*imin); dot_q6_k_q8k_avx2:
// (dx*d)*isum).  Every lane of the quad returns the value.
template <int FMT>
__device__ __forceinline__ float unit_block_value(const UnitLoad &L, int q, const Q4KScaleSel &S, bool ok,
                                                  const int32_t *xq32, const int16_t *bs, const int16_t *s16,
                                                  float dx) {
    // Computed unconditionally (a unit outside the tile holds clamped,
    // in-bounds bytes and is zeroed here), so no branch separates the units
    // and the scheduler can interleave their dot-product chains.
    if (FMT == F_Q4_K) {
        int isum, imin;
        Q4KLoad Q;
        Q.hdr = L.a;
        Q.a = L.b;
        Q.b = L.c;
        q4k_unit(Q, q, S, xq32, bs, isum, imin);
        isum = quad_sum_i32(ok ? isum : 0);
        imin = quad_sum_i32(ok ? imin : 0);
        float d = h2f(L.a.x & 0xFFFF), dmin = h2f(L.a.x >> 16);
        float t1 = d * (float)isum;
        float t2 = dmin * (float)imin;
        return dx * (t1 - t2);
    }
    Q6KLoad Q;
    Q.ql0 = L.a;
    Q.ql1 = L.b;
    Q.qh = L.c;
    Q.sc = L.sc;
    Q.d = L.dd;
    int isum = q6k_unit(Q, q, xq32, s16);
    isum = quad_sum_i32(ok ? isum : 0);
    return (dx * h2f(L.dd & 0xFFFF)) * (float)isum;
}

// K-quant GEMV.  A wave tile is TR rows x all nb blocks, 4*TR*nb <= 256
// quarter-block units, so every lane owns at most KQ_U = 4 units (unit u =
// lane + 64*i is quarter u&3 of block (u>>2)%nb of tile row (u>>2)/nb).  Each
// block's f32 value goes to a wave-private LDS row; lane r then sums row r
// serially in block order (the reference's accumulation order).  Waves are
// persistent over tiles and load the next tile's weights before computing the
// current one; the Q8_K activation is staged in LDS once per workgroup while
// the first tile's weights are in flight.  SWIGLU tiles hold TR gate rows
// followed by the same TR up rows.  FM: 1 = Q4_K only, 2 = Q6_K only, 3 = a
// launch mixing both (the format is uniform per tile).
#define KQ_U_MAX 4
#define KQ_XQ_IT (KMAX / 16 / 256)
// The Q8_K activation is staged in LDS with each 256-element block padded to
// 272 bytes: the four quads a ds_read_b128 pass serves read four different
// blocks at the same in-block offset, which would otherwise share banks.
#define KQ_XQ_STRIDE 68
#define KQ_XQ_WORDS (NB256_MAX * KQ_XQ_STRIDE > KQ_ACT_KMAX ? NB256_MAX * KQ_XQ_STRIDE : KQ_ACT_KMAX)

// sum(x*x) in dot_f32_avx2's order (as sumsq_avx2_order) from x staged
// transposed: xt[L * ld + c] = x[32c + L], so accumulator lane L (0..31) reads
// four steps of its chain per 16-byte read.  n % 32 == 0, n/32 % 4 == 0.
// red needs 33 floats; every thread receives the sum.
__device__ float kq_sumsq_t(const float *xt, int ld, int n, float *red) {
    const int C = n >> 5;
    if (threadIdx.x < 32) {
        const float *r = xt + threadIdx.x * ld;
        float acc = 0.0f;
        for (int c = 0; c < C; c += 4) {
            const float4 f = *(const float4 *)(r + c);
            acc = fmaf(f.x, f.x, acc);
            acc = fmaf(f.y, f.y, acc);
            acc = fmaf(f.z, f.z, acc);
            acc = fmaf(f.w, f.w, acc);
        }
        red[threadIdx.x] = acc;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float t[8];
#pragma unroll
        for (int l = 0; l < 8; l++) t[l] = (red[l] + red[8 + l]) + (red[16 + l] + red[24 + l]);
        red[32] = ((t[0] + t[4]) + (t[1] + t[5])) + ((t[2] + t[6]) + (t[3] + t[7]));
    }
    __syncthreads();
    return red[32];
}

// Q8_K of chunk c (16 consecutive elements v) into the LDS staging, exactly
// as quantize_row_q8k (src/simd.rs:5013-5101): a block's 16 chunks sit in 16
// consecutive lanes, which exchange the block maximum; the chunk's own sum is
// its per-16 sum and a lane pair's the per-32 bsum.  Every lane of the wave
// takes part (chunks past the end hold zeros and store nothing).
__device__ __forceinline__ void kq_quant_chunk(const float (&v)[16], int c, bool valid, int32_t *s_xq, float *s_dx,
                                               int16_t *s_bs, int16_t *s_s16) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = row_max16(amax);
    const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
    int sum = 0;
    uint32_t w4[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int q = max(-128, min(127, (int)__builtin_rintf(v[i] * id)));
        sum += q;
        w4[i >> 2] |= (uint32_t)(q & 0xFF) << (8 * (i & 3));
    }
    const int pair = sum + dpp_i<0xB1>(sum);  // quad_perm: the partner lane c ^ 1
    if (valid) {
        const int b = c >> 4;
        *(int4 *)(s_xq + b * KQ_XQ_STRIDE + (c & 15) * 4) = make_int4((int)w4[0], (int)w4[1], (int)w4[2], (int)w4[3]);
        s_s16[c] = (int16_t)sum;
        if ((c & 1) == 0) s_bs[c >> 1] = (int16_t)pair;
        if ((c & 15) == 0) s_dx[b] = amax * (1.0f / 127.0f);
    }
}

struct KqTile {
    GemvMat M;  // the tile's matrix (SWIGLU: the gate matrix)
    int row0, valid;
};

// Where lane's units sit in every tile of a launch: unit u = lane + 64*i is
// quarter u&3 of block (u>>2) % nb of tile row (u>>2) / nb.  The layout is
// the same for all tiles, so it is worked out once per wave.
template <int KQ_U>
struct KqGeo {
    int rrow[KQ_U];      // row offset from the tile's first row (SWIGLU up rows: from the up matrix's)
    int64_t roff[KQ_U];  // byte offset of the unit's block from the tile's first row
    int blk[KQ_U];   // block index
    int vidx[KQ_U];  // slot of the block value in the wave's LDS row buffer
    bool up[KQ_U];   // SWIGLU: the unit reads the up matrix
    bool in[KQ_U];   // the unit index is inside the tile
};
template <int FMT, bool SWIGLU, int KQ_U>
__device__ __forceinline__ KqGeo<KQ_U> kq_geo(int tr, int nb, int nbp, int64_t stride, int lane) {
    KqGeo<KQ_U> G;
    const int units = (SWIGLU ? 2 : 1) * tr * nb * 4;
#pragma unroll
    for (int i = 0; i < KQ_U; i++) {
        const int u = lane + 64 * i;
        const int rt = (u >> 2) / nb, b = (u >> 2) - rt * nb;
        G.up[i] = SWIGLU && rt >= tr;
        G.rrow[i] = G.up[i] ? rt - tr : rt;
        G.blk[i] = b;
        G.roff[i] = (int64_t)G.rrow[i] * stride + b * (FMT == F_Q4_K ? 144 : 210);
        G.vidx[i] = rt * nbp + b;
        G.in[i] = u < units;
    }
    return G;
}

// Row-split tiles (KQ_SPLIT): a tile is one row whose nb blocks are shared by
// the workgroup's four waves, bw = ceil(nb / 4) consecutive blocks each (one
// unit per lane), so a wide row (K = 14336: 56 blocks) runs with the
// one-unit geometry instead of four units per lane.
template <int FMT>
__device__ __forceinline__ KqGeo<1> kq_geo_split(int nb, int wave, int lane) {
    KqGeo<1> G;
    const int bw = (nb + 3) >> 2, b = wave * bw + (lane >> 2);
    G.up[0] = false;
    G.rrow[0] = 0;
    G.in[0] = (lane >> 2) < bw && b < nb;
    G.blk[0] = G.in[0] ? b : 0;
    G.vidx[0] = G.blk[0];
    G.roff[0] = (int64_t)G.blk[0] * (FMT == F_Q4_K ? 144 : 210);
    return G;
}

template <int FMT, bool SWIGLU, int KQ_U>
__device__ __forceinline__ void kq_load_tile(const GemvArgs &A, const KqTile &T, const KqGeo<KQ_U> &G,
                                             UnitLoad (&L)[KQ_U]) {
    // Every lane issues the same loads on every path (units past the tile or
    // the matrix read offset 0 and are discarded), so the compiler's vmcnt
    // bookkeeping stays exact and the next tile's loads stay in flight while
    // this tile computes.
    // All matrices of a K-quant launch share one row stride (same format and
    // K), so a unit's address is the tile's (scalar) row base plus its
    // precomputed per-lane offset.
    const int64_t base = (int64_t)T.row0 * A.m[0].row_stride;
#pragma unroll
    for (int i = 0; i < KQ_U; i++) {
        const int row = T.row0 + G.rrow[i];
        const bool up = G.up[i];
        const uint8_t *w = up ? A.m[1].w : T.M.w;
        const int rows = up ? A.m[1].rows : T.M.rows;
        const bool ok = T.valid && G.in[i] && row < rows;
        const int64_t off = ok ? base + G.roff[i] : 0;
        unit_load<FMT>(w + off, threadIdx.x & 3, L[i]);
    }
}

// Epilogue operands of a tile (lane r: row row0 + r), loaded before the next
// tile's weights so that waiting for them does not wait for those.  The loads
// are unconditional (clamped row, y standing in for a null bias).
struct KqEpi {
    float bias, y;
};
template <bool SWIGLU>
__device__ __forceinline__ KqEpi kq_epi_load(const KqTile &T, int lane) {
    KqEpi E = {0.0f, 0.0f};
    if (!SWIGLU) {
        const int row = min(T.row0 + lane, T.M.rows - 1);
        const float *bp = T.M.bias ? T.M.bias : T.M.y;
        E.bias = bp[row];
        E.y = T.M.y[row];
    }
    return E;
}

// Serial sum of n block values in block order (the reference's per-row
// accumulation), four per LDS read; p is 16-byte aligned.
__device__ __forceinline__ float kq_row_sum(const float *p, int n) {
    float acc = 0.0f;
    int b = 0;
    for (; b + 16 <= n; b += 16) {
        const float4 v0 = *(const float4 *)(p + b), v1 = *(const float4 *)(p + b + 4);
        const float4 v2 = *(const float4 *)(p + b + 8), v3 = *(const float4 *)(p + b + 12);
        acc += v0.x; acc += v0.y; acc += v0.z; acc += v0.w;
        acc += v1.x; acc += v1.y; acc += v1.z; acc += v1.w;
        acc += v2.x; acc += v2.y; acc += v2.z; acc += v2.w;
        acc += v3.x; acc += v3.y; acc += v3.z; acc += v3.w;
    }
    for (; b + 4 <= n; b += 4) {
        const float4 v = *(const float4 *)(p + b);
        acc += v.x;
        acc += v.y;
        acc += v.z;
        acc += v.w;
    }
    for (; b < n; b++) acc += p[b];
    return acc;
}

template <int FMT, bool SWIGLU, int KQ_U>
__device__ __forceinline__ void kq_compute_tile(const GemvArgs &A, const KqTile &T, const KqEpi &E,
                                                const KqGeo<KQ_U> &G, const Q4KScaleSel &S, int tr, int nb, int nbp,
                                                int lane, const UnitLoad (&L)[KQ_U], const int32_t *s_xq,
                                                const float *s_dx, const int16_t *s_bs, const int16_t *s_s16,
                                                float *s_v) {
    const int q = lane & 3;
#pragma unroll
    for (int i = 0; i < KQ_U; i++) {
        const int row = T.row0 + G.rrow[i];
        const bool ok = G.in[i] && row < (G.up[i] ? A.m[1].rows : T.M.rows);
        const int bb = ok ? G.blk[i] : 0;
        float v = unit_block_value<FMT>(L[i], q, S, ok, s_xq + bb * KQ_XQ_STRIDE, s_bs + bb * 8, s_s16 + bb * 16,
                                        s_dx[bb]);
        if (ok && q == 0) s_v[G.vidx[i]] = v;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < tr) {
        const GemvMat &M = T.M;
        const int row = T.row0 + lane;
        if (row < M.rows) {
            float acc = kq_row_sum(s_v + lane * nbp, nb);
            if (SWIGLU) {
                const float up = kq_row_sum(s_v + (tr + lane) * nbp, nb);
                M.y[row] = silu_mul_ref(acc, up);
            } else {
                if (M.bias) acc += E.bias;
                if (A.epi == EPI_ADD)
                    M.y[row] = E.y + acc;
                else
                    M.y[row] = acc;
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A row-split tile: every wave stores its blocks' values in the workgroup's
// row buffer (parity: the tile's, so the next tile's values go to the other
// half while this one is summed), then lane 0 of wave 0 sums the row serially
// in block order.  Every wave of the workgroup runs the same tiles, so the
// barrier is uniform.
template <int FMT>
__device__ __forceinline__ void kq_compute_split(const GemvArgs &A, const KqTile &T, const KqEpi &E,
                                                 const KqGeo<1> &G, const Q4KScaleSel &S, int nb, int wave, int lane,
                                                 int parity, const UnitLoad (&L)[1], const int32_t *s_xq,
                                                 const float *s_dx, const int16_t *s_bs, const int16_t *s_s16,
                                                 float *s_row) {
    const int q = lane & 3;
    const bool ok = G.in[0];
    const int bb = G.blk[0];
    const float v = unit_block_value<FMT>(L[0], q, S, ok, s_xq + bb * KQ_XQ_STRIDE, s_bs + bb * 8, s_s16 + bb * 16,
                                          s_dx[bb]);
    float *row = s_row + parity * 64;
    if (ok && q == 0) row[bb] = v;
    __syncthreads();
    if (wave == 0 && lane == 0 && T.row0 < T.M.rows) {
        float acc = kq_row_sum(row, nb);
        if (T.M.bias) acc += E.bias;
        T.M.y[T.row0] = A.epi == EPI_ADD ? E.y + acc : acc;
    }
}

template <bool SWIGLU, int KOFF = 0>
__device__ __forceinline__ KqTile kq_tile_info(const GemvArgs &A, int tile, int tr) {
    KqTile T;
    T.valid = tile < A.n_tiles;
    int mi = 0;
    if (!SWIGLU) {
#pragma unroll
        for (int t = 1; t < GEMV_MAX_MATS; t++)
            if (t < A.n_mats && tile >= A.m[t].tile_begin) mi = t;
    }
    T.M = mat_sel<KOFF>(A, mi);
    T.row0 = (tile - T.M.tile_begin) * tr;
    return T;
}

// FMT: every matrix of the launch has this format (Q4_K or Q6_K).  KQ_U:
// units per lane (a wave tile is 64*KQ_U quarter-block units).
// XQW: words of the activation staging (NORM2 stages K + 128 floats of x)
template <int XQW>
struct KqSharedT {
    __align__(16) int32_t xq[XQW];
    float red[40];
    float dx[NB256_MAX];
    int16_t bs[NB32_MAX];
    int16_t s16[KMAX / 16];
    __align__(16) float v[4][64];  // per wave: the tile's block values (row-split tiles: v[0..1] is the
                                   // workgroup's row buffer, two halves by tile parity)
};
using KqShared = KqSharedT<KQ_XQ_WORDS>;
template <int ACT>
using KqSharedFor = typename std::conditional<ACT == KQ_ACT_NORM2, KqSharedT<8192 + 128>, KqShared>::type;

// One workgroup's share of a launch: workgroup blk of the nblk that serve
// A's tiles (the whole grid for a one-group launch).
template <int FMT, bool SWIGLU, int KQ_U, int ACT, int KOFF, bool SPLIT = false, class SHT = KqShared>
__device__ __forceinline__ void kq_run(const GemvArgs &A, int blk, int nblk, SHT &SH) {
    static_assert(ACT != KQ_ACT_NORM2 || sizeof(SH.xq) >= (8192 + 128) * 4, "NORM2 stages up to 8320 floats");
    constexpr bool NORMA = ACT == KQ_ACT_NORM || ACT == KQ_ACT_NORM2;
    constexpr bool DENA = ACT == KQ_ACT_DEN || ACT == KQ_ACT_DEN2;
    constexpr int CH = (ACT == KQ_ACT_NORM2 || ACT == KQ_ACT_DEN2) ? 2 : 1;  // 16-element chunks per thread
    static_assert(!SPLIT || (KQ_U == 1 && !SWIGLU), "row-split tiles: one unit per lane, plain rows");
    int32_t *s_xq = SH.xq;
    float *s_red = SH.red;
    float *s_dx = SH.dx;
    int16_t *s_bs = SH.bs;
    int16_t *s_s16 = SH.s16;
    float(*s_v)[64] = SH.v;

    const int K = A.K, nb = K >> 8, nbp = (nb + 3) & ~3;
    const int tr = A.tile_rows;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps tile math scalar
    // Prologue: the activation's loads first, then the first two tiles'
    // weights and epilogue operands, so that staging the activation in LDS
    // waits only for its own loads and both tiles are in flight from the
    // start.  Each tile's epilogue loads follow its weights: computing a tile
    // then waits for exactly the loads issued before the next tile's.
    static_assert(KQ_XQ_IT == 4, "staging below is written for K <= 16384");
    const int n16 = K >> 4;
    const int nbs = K >> 8;   // int4 chunks of bsums (8 per 256)
    const int ns16 = K >> 7;  // int4 chunks of sums16 (16 per 256)
    int4 x0, x1, x2, x3, bsr, s16r;
    float dxr;
    float4 xf[NORMA ? 8 * CH : 1];  // chunk tid + 256 h of x, then of w (NORM), per h < CH
    float4 xd[DENA ? 4 * CH : 1];   // chunk tid + 256 h (DEN)
    float4 xq4[ACT == KQ_ACT_QUANT ? 16 : 1];  // chunks tid + 256 r, r < 4 (QUANT)
    float dd[CH];
    if (ACT == KQ_ACT_XQ) {
        const int4 *src = (const int4 *)A.xq.qs;
        x0 = src[min(tid, n16 - 1)];
        x1 = src[min(tid + 256, n16 - 1)];
        x2 = src[min(tid + 512, n16 - 1)];
        x3 = src[min(tid + 768, n16 - 1)];
        bsr = ((const int4 *)A.xq.bsums)[min(tid, nbs - 1)];
        s16r = ((const int4 *)A.xq.sums16)[min(tid, ns16 - 1)];
        dxr = A.xq.d[min(tid, nb - 1)];
    } else if (NORMA) {
#pragma unroll
        for (int h = 0; h < CH; h++) {
            const int c = min(tid + 256 * h, n16 - 1);
#pragma unroll
            for (int i = 0; i < 4; i++) xf[8 * h + i] = ((const float4 *)A.act_x)[4 * c + i];
#pragma unroll
            for (int i = 0; i < 4; i++) xf[8 * h + 4 + i] = ((const float4 *)A.act_w)[4 * c + i];
        }
    } else if (DENA) {
#pragma unroll
        for (int h = 0; h < CH; h++) {
            const int c = min(tid + 256 * h, n16 - 1);
#pragma unroll
            for (int i = 0; i < 4; i++) xd[4 * h + i] = ((const float4 *)A.act_x)[4 * c + i];
            dd[h] = A.act_den[(16 * c) / A.act_group];
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int c = min(tid + 256 * r, n16 - 1);
#pragma unroll
            for (int i = 0; i < 4; i++) xq4[4 * r + i] = ((const float4 *)A.act_x)[4 * c + i];
        }
    }

    // the activation's loads are issued before the tile geometry's arithmetic
    __builtin_amdgcn_sched_barrier(0);
    // row-split: the workgroup's waves share each tile (one row)
    const int step = SPLIT ? nblk : nblk * 4;
    int tile = SPLIT ? blk : blk * 4 + wave;
    KqGeo<KQ_U> G;
    if constexpr (SPLIT) G = kq_geo_split<FMT>(nb, wave, lane);
    else G = kq_geo<FMT, SWIGLU, KQ_U>(tr, nb, nbp, A.m[0].row_stride, lane);
    const Q4KScaleSel S = q4k_scale_sel(lane & 3);

    UnitLoad L0[KQ_U], L1[KQ_U];
    KqTile T0 = kq_tile_info<SWIGLU, KOFF>(A, tile, tr);
    kq_load_tile<FMT, SWIGLU, KQ_U>(A, T0, G, L0);
    KqEpi E0 = kq_epi_load<SWIGLU>(T0, lane);
    KqTile T1 = kq_tile_info<SWIGLU, KOFF>(A, tile + step, tr);
    KqEpi E1;
    if (!NORMA) {
        kq_load_tile<FMT, SWIGLU, KQ_U>(A, T1, G, L1);
        E1 = kq_epi_load<SWIGLU>(T1, lane);
    }
    if (ACT == KQ_ACT_XQ) {
        // 16-byte chunk c of the activation goes to block c/16, padded stride
        int4 *dst = (int4 *)s_xq;
        const int d0 = (tid >> 4) * (KQ_XQ_STRIDE / 4) + (tid & 15);
        if (tid < n16) dst[d0] = x0;
        if (tid + 256 < n16) dst[d0 + 16 * (KQ_XQ_STRIDE / 4)] = x1;
        if (tid + 512 < n16) dst[d0 + 32 * (KQ_XQ_STRIDE / 4)] = x2;
        if (tid + 768 < n16) dst[d0 + 48 * (KQ_XQ_STRIDE / 4)] = x3;
        if (tid < nbs) ((int4 *)s_bs)[tid] = bsr;
        if (tid < ns16) ((int4 *)s_s16)[tid] = s16r;
        if (tid < nb) s_dx[tid] = dxr;
    } else if (NORMA) {
        // rms_norm_into (src/model.rs:5429-5437): x staged as f32 in the
        // quant buffer, sum of squares in the reference's AVX2 order, then
        // (x * scale) * w per element and Q8_K of the result
        // x and w (this thread's 16-element chunks, loaded ahead of the first
        // tile's weights) stay in registers; x is also staged transposed
        // (element 32c + L at L*ld + c) for the sum of squares
        float *s_xt = (float *)s_xq;
        const int ld = (K >> 5) + 4;
#pragma unroll
        for (int h = 0; h < CH; h++) {
            const int ci = tid + 256 * h;
            if (ci < n16) {
                const int c = ci >> 1, l0 = 16 * (ci & 1);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    s_xt[(l0 + 4 * i + 0) * ld + c] = xf[8 * h + i].x;
                    s_xt[(l0 + 4 * i + 1) * ld + c] = xf[8 * h + i].y;
                    s_xt[(l0 + 4 * i + 2) * ld + c] = xf[8 * h + i].z;
                    s_xt[(l0 + 4 * i + 3) * ld + c] = xf[8 * h + i].w;
                }
            }
        }
        kq_load_tile<FMT, SWIGLU, KQ_U>(A, T1, G, L1);
        E1 = kq_epi_load<SWIGLU>(T1, lane);
        __syncthreads();
        const float ss = kq_sumsq_t(s_xt, ld, K, s_red);
        const float scale = 1.0f / sqrtf(ss / (float)K + A.act_eps);
        float v[CH][16];
#pragma unroll
        for (int h = 0; h < CH; h++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 xv = xf[8 * h + i];
                const float4 wv = xf[8 * h + 4 + i];
                v[h][4 * i + 0] = xv.x * scale * wv.x;
                v[h][4 * i + 1] = xv.y * scale * wv.y;
                v[h][4 * i + 2] = xv.z * scale * wv.z;
                v[h][4 * i + 3] = xv.w * scale * wv.w;
            }
        __syncthreads();  // every read of the f32 staging precedes the quant stores over it
#pragma unroll
        for (int h = 0; h < CH; h++) kq_quant_chunk(v[h], tid + 256 * h, tid + 256 * h < n16, s_xq, s_dx, s_bs, s_s16);
    } else if (ACT == KQ_ACT_QUANT) {
        // the standalone quantize_q8k_kernel's values, chunk by chunk
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[4 * i + 0] = xq4[4 * r + i].x;
                v[4 * i + 1] = xq4[4 * r + i].y;
                v[4 * i + 2] = xq4[4 * r + i].z;
                v[4 * i + 3] = xq4[4 * r + i].w;
            }
            kq_quant_chunk(v, tid + 256 * r, tid + 256 * r < n16, s_xq, s_dx, s_bs, s_s16);
        }
    } else {
        // attention normalisation (out *= 1/den where den > 0, as the
        // reference's final scale) and Q8_K
#pragma unroll
        for (int h = 0; h < CH; h++) {
            float v[16];
            const float d = dd[h];
            const float inv = d > 0.0f ? 1.0f / d : 1.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 a = xd[4 * h + i];
                v[4 * i + 0] = d > 0.0f ? a.x * inv : a.x;
                v[4 * i + 1] = d > 0.0f ? a.y * inv : a.y;
                v[4 * i + 2] = d > 0.0f ? a.z * inv : a.z;
                v[4 * i + 3] = d > 0.0f ? a.w * inv : a.w;
            }
            kq_quant_chunk(v, tid + 256 * h, tid + 256 * h < n16, s_xq, s_dx, s_bs, s_s16);
        }
    }
    __syncthreads();
    if (ACT != KQ_ACT_XQ && A.act_store && blk == 0) {
        // the same vector for a later launch that consumes it as is
        for (int c = tid; c < n16; c += 256) ((int4 *)A.xq.qs)[c] = ((const int4 *)s_xq)[(c >> 4) * (KQ_XQ_STRIDE / 4) + (c & 15)];
        if (tid < nbs) ((int4 *)A.xq.bsums)[tid] = ((const int4 *)s_bs)[tid];
        if (tid < ns16) ((int4 *)A.xq.sums16)[tid] = ((const int4 *)s_s16)[tid];
        if (tid < nb) A.xq.d[tid] = s_dx[tid];
    }

    if constexpr (SPLIT) {
        while (T0.valid) {
            kq_compute_split<FMT>(A, T0, E0, G, S, nb, wave, lane, 0, L0, s_xq, s_dx, s_bs, s_s16, s_v[0]);
            tile += step;
            if (!T1.valid) break;
            T0 = kq_tile_info<SWIGLU, KOFF>(A, tile + step, tr);
            kq_load_tile<FMT, SWIGLU, KQ_U>(A, T0, G, L0);
            E0 = kq_epi_load<SWIGLU>(T0, lane);
            kq_compute_split<FMT>(A, T1, E1, G, S, nb, wave, lane, 1, L1, s_xq, s_dx, s_bs, s_s16, s_v[0]);
            tile += step;
            if (!T0.valid) break;
            T1 = kq_tile_info<SWIGLU, KOFF>(A, tile + step, tr);
            kq_load_tile<FMT, SWIGLU, KQ_U>(A, T1, G, L1);
            E1 = kq_epi_load<SWIGLU>(T1, lane);
        }
        return;
    }
    while (T0.valid) {
        kq_compute_tile<FMT, SWIGLU, KQ_U>(A, T0, E0, G, S, tr, nb, nbp, lane, L0, s_xq, s_dx, s_bs, s_s16,
                                           s_v[wave]);
        tile += step;
        if (!T1.valid) break;
        T0 = kq_tile_info<SWIGLU, KOFF>(A, tile + step, tr);
        kq_load_tile<FMT, SWIGLU, KQ_U>(A, T0, G, L0);
        E0 = kq_epi_load<SWIGLU>(T0, lane);
        kq_compute_tile<FMT, SWIGLU, KQ_U>(A, T1, E1, G, S, tr, nb, nbp, lane, L1, s_xq, s_dx, s_bs, s_s16,
                                           s_v[wave]);
        tile += step;
        if (!T0.valid) break;
        T1 = kq_tile_info<SWIGLU, KOFF>(A, tile + step, tr);
        kq_load_tile<FMT, SWIGLU, KQ_U>(A, T1, G, L1);
        E1 = kq_epi_load<SWIGLU>(T1, lane);
    }
}

template <int FMT, bool SWIGLU, int KQ_U, int ACT, bool SPLIT = false>
__global__ __launch_bounds__(256) void gemv_kq_kernel(GemvArgs A) {
    __shared__ KqSharedFor<ACT> sh;
    kq_run<FMT, SWIGLU, KQ_U, ACT, 0, SPLIT>(A, blockIdx.x, gridDim.x, sh);
}

// Two launch groups of different formats that build the same activation in
// their prologue (a layer's wq/wk in Q4_K and wv in Q6_K): workgroups below
// grid_a serve A, the rest B, so the layer's q/k/v products take one launch.
// Every tile is computed exactly as in the one-group kernel.
template <int FA, int UA, int FB, int UB, int ACT>
__global__ __launch_bounds__(256) void gemv_kq2_kernel(GemvArgs A, GemvArgs B, int grid_a) {
    __shared__ KqSharedFor<ACT> sh;
    if ((int)blockIdx.x < grid_a)
        kq_run<FA, false, UA, ACT, 0>(A, blockIdx.x, grid_a, sh);
    else
        kq_run<FB, false, UB, ACT, KARG_SECOND>(B, blockIdx.x - grid_a, gridDim.x - grid_a, sh);
}

// ---- 32-element-block formats: Q8_0 (int / f32) and MXFP4 --------------------
#define B32_VMAX 8192  // floats of per-row staging in LDS

__constant__ float kMxfp4Lut[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

// Both FP4 values of byte u of w (low nibble first), each times scale:
// gfx950's v_cvt_scalef32_pk_f32_fp4.
typedef float fp4x2_f32 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ fp4x2_f32 fp4x2_scaled(uint32_t w, float scale, int u) {
    switch (u) {
    case 0: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 0);
    case 1: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 1);
    case 2: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 2);
    default: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 3);
    }
}

// kMxfp4Lut[n] without a memory access: magnitudes 0 and 0.5 for n & 7 < 2,
// else exponent 126 + (n & 7) / 2 with the low bit as the one mantissa bit;
// bit 3 is the sign (n = 8 gives -0).
__device__ __forceinline__ float mxfp4_nibble(uint32_t n) {
    const uint32_t v = n & 7u;
    const float mag = v < 2u ? (float)v * 0.5f : __builtin_bit_cast(float, (v << 22) + 0x3F000000u);
    return (n & 8u) ? -mag : mag;
}

__device__ __forceinline__ float mxfp4_scale(uint32_t e) {
    // 2^(e-127) as an exact power of two (e = 0 is the subnormal 2^-127).
    if (e == 0) return __builtin_bit_cast(float, 0x00400000u);
    return __builtin_bit_cast(float, e << 23);
}

// Q8_0, K % 256 == 0: reproduces dot_q8_0_q8k_avx2 (src/simd.rs:7184-7210):
// eight lane accumulators acc_j = fma(dx*d_b, s_{b,j}, acc_j) over blocks in
// order, s_{b,j} = exact int dot of bytes 4j..4j+3, then the hsum_avx tree.
// A persistent grid of independent waves.  A wave tile is 8 rows; the wave
// walks its tiles' rows in chunks of Q8P_CH blocks (items), the next item's
// weights in flight while it works on the current one:
//   owner step: lane (r, j) holds blocks 8j..8j+7 of the chunk of row r
//     (272 bytes = 17 aligned 16-byte loads; one Q8_K block of x, one dx)
//     and computes c_b = dx * d_b and s_{b,i} (i < 8) for them;
//   chain step: through a wave-private LDS transpose, lane (r, j) runs
//     accumulator j of row r over the chunk's blocks in order,
//     acc = fma(c_b, s_{b,j}, acc);
// after a row's last chunk, hsum_avx over the eight lanes.
// ACT: the Q8_K activation from memory (KQ_ACT_XQ) or built in the prologue
// as in the K-quant kernel (RMSNorm, attention normalisation or plain Q8_K,
// the same arithmetic), staged in the K-quant kernel's padded layout.
// SWIGLU: a tile is rows row0..row0+3 of the gate matrix (lanes r < 4) and of
// the up matrix (r >= 4); y = silu(gate) * up.
#define Q8P_CH 64   // blocks of a row per item: 8 lanes x 272 bytes
#define Q8P_PAD 68  // floats per (row, accumulator) line of the transpose
template <int ACT>
__device__ __forceinline__ void q8p_build_act(const GemvArgs &A, KqShared &sh, int nt) {
    const int K = A.K, n16 = K >> 4, tid = threadIdx.x;
    if (ACT == KQ_ACT_XQ) {
        const int4 *src = (const int4 *)A.xq.qs;
        int4 *dst = (int4 *)sh.xq;
        for (int c = tid; c < n16; c += nt) dst[(c >> 4) * (KQ_XQ_STRIDE / 4) + (c & 15)] = src[c];
        for (int b = tid; b < (K >> 8); b += nt) sh.dx[b] = A.xq.d[b];
        return;
    }
    float scale = 1.0f;
    if (ACT == KQ_ACT_NORM) {
        // rms_norm_into (src/model.rs:5429-5437): the sum of squares in the
        // reference's AVX2 order from x staged transposed (element 32c + L
        // at L*ld + c), then (x * scale) * w per element
        float *s_xt = (float *)sh.xq;
        const int ld = (K >> 5) + 4;
        for (int c = tid; c < n16; c += nt) {
            const int cc = c >> 1, l0 = 16 * (c & 1);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 xv = ((const float4 *)A.act_x)[4 * c + i];
                s_xt[(l0 + 4 * i + 0) * ld + cc] = xv.x;
                s_xt[(l0 + 4 * i + 1) * ld + cc] = xv.y;
                s_xt[(l0 + 4 * i + 2) * ld + cc] = xv.z;
                s_xt[(l0 + 4 * i + 3) * ld + cc] = xv.w;
            }
        }
        __syncthreads();
        const float ss = kq_sumsq_t(s_xt, ld, K, sh.red);  // ends with a barrier after its reads
        scale = 1.0f / sqrtf(ss / (float)K + A.act_eps);
    }
    // chunk c = 16 elements; a 256-block's 16 chunks sit in 16 consecutive
    // lanes (nt is a multiple of 64), every lane takes part in each pass
    for (int base = 0; base < n16; base += nt) {
        const int c = base + tid, cl = min(c, n16 - 1);
        float v[16];
        float dd = 0.0f;
        if (ACT == KQ_ACT_DEN) dd = A.act_den[(16 * cl) / A.act_group];
        const float inv = dd > 0.0f ? 1.0f / dd : 1.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 xv = ((const float4 *)A.act_x)[4 * cl + i];
            const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
            float4 wv = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            if (ACT == KQ_ACT_NORM) wv = ((const float4 *)A.act_w)[4 * cl + i];
            const float ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (ACT == KQ_ACT_NORM) v[4 * i + e] = xs[e] * scale * ws[e];
                else if (ACT == KQ_ACT_DEN) v[4 * i + e] = dd > 0.0f ? xs[e] * inv : xs[e];
                else v[4 * i + e] = xs[e];
            }
        }
        // (NORM: the staging's last reads precede kq_sumsq_t's barrier, so the
        // quant stores may overwrite it)
        kq_quant_chunk(v, c, c < n16, sh.xq, sh.dx, sh.bs, sh.s16);
    }
}

template <int WAVES, int ACT, bool SWIGLU>
__global__ __launch_bounds__(64 * WAVES) void gemv_q8_0_pipe_kernel(GemvArgs A) {
    __shared__ KqShared sh;
    __shared__ __align__(16) float s_s[WAVES][8][8][Q8P_PAD];  // [wave][row][accumulator][block]: s
    __shared__ __align__(16) float s_c[WAVES][8][Q8P_CH];      // [wave][row][block]: c
    const int K = A.K, nb = K >> 5, nch = (nb + Q8P_CH - 1) / Q8P_CH;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    q8p_build_act<ACT>(A, sh, 64 * WAVES);
    __syncthreads();
    const int r = lane >> 3, j = lane & 7;
    // the tile's rows: 8 of one matrix, or (SWIGLU) 4 of the gate and the
    // same 4 of the up matrix
    constexpr int TR = SWIGLU ? 4 : 8;
    const int rr = SWIGLU ? (r & 3) : r;
    const int gw = blockIdx.x * WAVES + wave, nw = gridDim.x * WAVES;
    const int my_tiles = gw < A.n_tiles ? (A.n_tiles - 1 - gw) / nw + 1 : 0;
    const int n_items = my_tiles * nch;
    auto mat_of = [&](int tile) {
        if (SWIGLU) return mat_sel(A, 0);
        int mi = 0;
#pragma unroll
        for (int t = 1; t < GEMV_MAX_MATS; t++)
            if (t < A.n_mats && tile >= A.m[t].tile_begin) mi = t;
        return mat_sel(A, mi);
    };
    // (SWIGLU) the up matrix's bytes for lanes r >= 4; both share rows and stride
    const uint8_t *w_up = SWIGLU ? A.m[1].w : nullptr;
    // item i: tile gw + (i / nch) * nw, chunk i % nch; loads are clamped in
    // bounds and unconditional, so the vmcnt bookkeeping stays exact
    auto load = [&](int i, uint4 (&w)[17]) {
        const int ii = min(i, n_items - 1);
        const int tile = gw + (ii / nch) * nw, ch = ii % nch;
        const GemvMat M = mat_of(tile);
        const int row = min((tile - M.tile_begin) * TR + rr, M.rows - 1);
        const int b0 = min(ch * Q8P_CH + 8 * j, nb - 8);
        const uint8_t *wm = (SWIGLU && r >= 4) ? w_up : M.w;
        const uint4 *p = (const uint4 *)(wm + (int64_t)row * M.row_stride + (int64_t)b0 * 34);
#pragma unroll
        for (int q = 0; q < 17; q++) w[q] = p[q];
    };
    float acc = 0.0f;
    auto process = [&](int i, const uint4 (&w)[17]) {
        const int tile = gw + (i / nch) * nw, ch = i % nch;
        const GemvMat M = mat_of(tile);
        const int row = (tile - M.tile_begin) * TR + rr;
        const int b0 = ch * Q8P_CH + 8 * j;
        uint32_t wd[68];
        __builtin_memcpy(wd, w, sizeof(wd));
        const int bx = min(b0, nb - 8);
        const float dx = sh.dx[bx >> 3];
        // x of this lane's 256-block in the padded staging
        const int32_t *xb = sh.xq + (bx >> 3) * KQ_XQ_STRIDE;
        float sv[8][8];  // [accumulator][block]
        float cv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            // block k at byte 34k: even k start dword-aligned (d, then quants 2
            // bytes off), odd k start 2 bytes in (quants aligned)
            const int m = 17 * (k >> 1);
            uint32_t q[8];
            uint16_t d;
            if ((k & 1) == 0) {
                d = (uint16_t)(wd[m] & 0xFFFFu);
#pragma unroll
                for (int t = 0; t < 8; t++) q[t] = __builtin_amdgcn_alignbyte(wd[m + t + 1], wd[m + t], 2);
            } else {
                d = (uint16_t)(wd[m + 8] >> 16);
#pragma unroll
                for (int t = 0; t < 8; t++) q[t] = wd[m + 9 + t];
            }
            const int4 *xp = (const int4 *)(xb + k * 8);
            const int4 x0 = xp[0], x1 = xp[1];
            sv[0][k] = (float)sdot4(q[0], x0.x, 0);
            sv[1][k] = (float)sdot4(q[1], x0.y, 0);
            sv[2][k] = (float)sdot4(q[2], x0.z, 0);
            sv[3][k] = (float)sdot4(q[3], x0.w, 0);
            sv[4][k] = (float)sdot4(q[4], x1.x, 0);
            sv[5][k] = (float)sdot4(q[5], x1.y, 0);
            sv[6][k] = (float)sdot4(q[6], x1.z, 0);
            sv[7][k] = (float)sdot4(q[7], x1.w, 0);
            cv[k] = dx * h2f(d);
        }
        float *ss = &s_s[wave][r][0][8 * j];
#pragma unroll
        for (int t = 0; t < 8; t++) {
            *(float4 *)(ss + t * Q8P_PAD) = make_float4(sv[t][0], sv[t][1], sv[t][2], sv[t][3]);
            *(float4 *)(ss + t * Q8P_PAD + 4) = make_float4(sv[t][4], sv[t][5], sv[t][6], sv[t][7]);
        }
        float *sc = &s_c[wave][r][8 * j];
        *(float4 *)sc = make_float4(cv[0], cv[1], cv[2], cv[3]);
        *(float4 *)(sc + 4) = make_float4(cv[4], cv[5], cv[6], cv[7]);
        // the wave's transpose writes are complete before any lane reads them
        RH_WAIT_LGKM0();
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
        const int nbc = min(Q8P_CH, nb - ch * Q8P_CH);  // a multiple of 8
        const float *ps = &s_s[wave][r][j][0], *pc = &s_c[wave][r][0];
        for (int b = 0; b < nbc; b += 8) {
            const float4 s0 = *(const float4 *)(ps + b), s1 = *(const float4 *)(ps + b + 4);
            const float4 c0 = *(const float4 *)(pc + b), c1 = *(const float4 *)(pc + b + 4);
            acc = fmaf(c0.x, s0.x, acc);
            acc = fmaf(c0.y, s0.y, acc);
            acc = fmaf(c0.z, s0.z, acc);
            acc = fmaf(c0.w, s0.w, acc);
            acc = fmaf(c1.x, s1.x, acc);
            acc = fmaf(c1.y, s1.y, acc);
            acc = fmaf(c1.z, s1.z, acc);
            acc = fmaf(c1.w, s1.w, acc);
        }
        // the chain's reads are done before the next item's writes
        RH_WAIT_LGKM0();
        asm volatile("" ::: "memory");
        if (ch == nch - 1) {
            // hsum_avx: t_i = a_i + a_{i+4}; ((t0+t1) + (t2+t3))
            const float t = acc + __shfl_xor(acc, 4, 64);
            const float u = t + __shfl_xor(t, 1, 64);
            float v = u + __shfl_xor(u, 2, 64);
            if (SWIGLU) {
                // the up row's value from the lane four rows on
                const float up = __shfl(v, lane + 32, 64);
                if (j == 0 && r < 4 && row < M.rows) M.y[row] = silu_mul_ref(v, up);
            } else if (j == 0 && row < M.rows) {
                if (M.bias) v += M.bias[row];
                if (A.epi == EPI_ADD)
                    M.y[row] += v;
                else
                    M.y[row] = v;
            }
            acc = 0.0f;
        }
    };
    if (n_items <= 0) return;
    uint4 w0[17], w1[17];
    load(0, w0);
    for (int i = 0; i < n_items; i += 2) {
        load(i + 1, w1);
        process(i, w0);
        if (i + 1 >= n_items) break;
        load(i + 2, w0);
        process(i + 1, w1);
    }
}

// Q8_0 rows with f32 activations (dot_q8_0_f32_avx2, src/simd.rs:6671-6692),
// bit-identical: eight accumulators per row, acc_j = fma(d*q, x, acc_j) over
// elements 32b + 8i + j (block b outer, group i inner), then hsum_avx
// ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)); eight lanes per row (lane j is
// accumulator j), eight rows per wave.  A workgroup is one wave and one tile
// of 8 rows; the activation (the matrix's own, else the launch's) is staged
// in LDS.  The tile's bytes arrive in chunks of 32 blocks (8 rows x 1088
// bytes = 544 aligned 16-byte pieces, piece f = row * 68 + p) by 9 coalesced
// direct global->LDS loads into a double-buffered chunk, the next chunk's
// loads in flight while this one is summed; each lane then reads its
// block's scale (2 bytes) and its four quants (bytes 8i + j) from LDS.
#define Q8F_C 32  // blocks per chunk
template <bool NORM>
__global__ __launch_bounds__(64) void gemv_q8_0_f32x_kernel(GemvArgs A) {
    extern __shared__ float s_x[];  // [K]
    __shared__ __align__(16) uint4 s_w[2][9 * 64];
    const int K = A.K, nb = K >> 5, lane = threadIdx.x;
    const int tile = blockIdx.x;
    int mi = 0;
#pragma unroll
    for (int t = 1; t < GEMV_MAX_MATS; t++)
        if (t < A.n_mats && tile >= A.m[t].tile_begin) mi = t;
    const GemvMat M = mat_sel(A, mi);
    const float *xs = M.x ? M.x : A.x;
    const uint8_t *w = M.w;
    const float *bias = M.bias;
    if (M.sel) {
        const int64_t e = *M.sel;
        w += e * M.sel_w;
        if (bias) bias += e * M.sel_b;
    }
    const int row0 = (tile - M.tile_begin) * 8;
    const int64_t stride = M.row_stride;  // a multiple of 16 that holds nb * 34 bytes
    const int nch = (nb + Q8F_C - 1) / Q8F_C;
    auto issue_chunk = [&](int c, int buf) {
#pragma unroll
        for (int i = 0; i < 9; i++) {
            const int f = min(64 * i + lane, 8 * 68 - 1), r = f / 68, p = f - 68 * r;
            const int rr = min(row0 + r, M.rows - 1);
            const int64_t o = min((int64_t)(Q8F_C * 34 * c + 16 * p), stride - 16);
            dma16(w + (int64_t)rr * stride + o, &s_w[buf][64 * i]);
        }
    };
    issue_chunk(0, 0);
    if constexpr (NORM) {
        // rms_norm_into (src/model.rs:5429-5437) over the staged x, as
        // rmsnorm_row computes it; the weights (K <= 3072: twelve float4 per
        // lane) are loaded with x, before the sum of squares
        __shared__ float red[40];
        const int k4 = K >> 2;
        float4 wv[12], xv[12];
#pragma unroll
        for (int k = 0; k < 12; k++) {
            const int i4 = min(lane + 64 * k, k4 - 1);
            xv[k] = ((const float4 *)xs)[i4];
            wv[k] = ((const float4 *)A.norm_w)[i4];
        }
#pragma unroll
        for (int k = 0; k < 12; k++)
            if (lane + 64 * k < k4) ((float4 *)s_x)[lane + 64 * k] = xv[k];
        __syncthreads();
        const float ss = sumsq_avx2_order(s_x, K, red);
        const float scale = 1.0f / sqrtf(ss / (float)K + A.norm_eps);
#pragma unroll
        for (int k = 0; k < 12; k++) {
            const int i4 = lane + 64 * k;
            if (i4 < k4) {
                const float4 x4 = xv[k], w4 = wv[k];
                const float4 o = make_float4(x4.x * scale * w4.x, x4.y * scale * w4.y, x4.z * scale * w4.z,
                                             x4.w * scale * w4.w);
                ((float4 *)s_x)[i4] = o;
                if (blockIdx.x == 0) ((float4 *)A.norm_out)[i4] = o;
            }
        }
    } else {
        for (int i = 4 * lane; i < K; i += 256) *(float4 *)(s_x + i) = *(const float4 *)(xs + i);
    }
    const int j = lane & 7, rr = lane >> 3;
    const int row = row0 + rr;
    const bool ok = row < M.rows;
    float acc = 0.0f;
    for (int c = 0; c < nch; c++) {
        RH_WAIT_VM(0);
        __syncthreads();  // chunk c (and x) in LDS; every read of chunk c - 1 done
        if (c + 1 < nch) issue_chunk(c + 1, (c + 1) & 1);
        const uint8_t *rb = (const uint8_t *)&s_w[c & 1][0] + rr * (Q8F_C * 34);
        const int nbc = min(Q8F_C, nb - Q8F_C * c);
        for (int lb = 0; lb < nbc; lb++) {
            const uint8_t *blk = rb + 34 * lb;
            const float d = h2f(*(const uint16_t *)blk);
            const float *xb = s_x + (Q8F_C * c + lb) * 32 + j;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float q = (float)(int)(int8_t)blk[2 + 8 * i + j];
                acc = fmaf(d * q, xb[8 * i], acc);
            }
        }
    }
    const float t = acc + __shfl_xor(acc, 4, 64);
    const float u = t + __shfl_xor(t, 1, 64);
    float out = u + __shfl_xor(u, 2, 64);
    if (ok && j == 0) {
        if (bias) out += bias[row];
        if (A.epi == EPI_ADD)
            M.y[row] += out;
        else
            M.y[row] = out;
    }
}

// MXFP4 rows in dot_mxfp4_f32_scalar's order (src/simd.rs:5886-5902): one
// running sum per row over the elements in order, each term
// (lut[nibble] * scale) * x.  The sum is a dependent chain of K adds, so a
// row is one lane's work; the terms are independent.  A workgroup of
// 1 + MXP waves serves 64 rows of one matrix: waves 1..MXP compute the terms
// of one 32-element block each (lane = row) into an LDS ring, wave 0 adds
// them in order (lane = row), eight LDS reads and 32 adds per block.  One
// barrier per group of MXP blocks: the adder reads group j while the
// producers write group j + 1 into the ring's other half.
#define MXP 4   // producer waves
#define MX_D 4  // groups of block loads in flight per producer
typedef const __attribute__((address_space(4))) float *const_f32_ptr;
// Barrier that waits only for this wave's LDS operations (global loads stay in
// flight across it); the compiler fences keep memory accesses from moving
// across the barrier.
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt/expcnt unrestricted
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Ring layout: slot (block % 2P), 4-term group g (0..7) of the block, row r:
// one 16-byte read or write of a group by the wave's 64 rows covers 1 KB of
// consecutive LDS, every bank four times, the conflict-free minimum.
template <int P>
__global__ __launch_bounds__(64 * (P + 1)) void gemv_mxfp4_serial_kernel(
    GemvArgs A) {
    constexpr int NT = 64 * (P + 1), SLOTS = 2 * P;
    __shared__ __align__(16) float s_t[SLOTS][64 * 32];  // [slot][8 groups][row][4 terms]
    __shared__ float s_lut[16];
    const int K = A.K, nb = K >> 5, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = blockIdx.x;
    int mi = 0;
#pragma unroll
    for (int t = 1; t < GEMV_MAX_MATS; t++)
        if (t < A.n_mats && tile >= A.m[t].tile_begin) mi = t;
    const GemvMat M = mat_sel(A, mi);
    const float *xs = M.x ? M.x : A.x;
    if (tid < 16) s_lut[tid] = kMxfp4Lut[tid];
    const uint8_t *w = M.w;
    const float *bias = M.bias;
    if (M.sel) {
        const int64_t e = *M.sel;
        w += e * M.sel_w;
        if (bias) bias += e * M.sel_b;
    }
    const int row = (tile - M.tile_begin) * 64 + lane;
    const bool live = row < M.rows;
    const uint8_t *rp = w + (int64_t)(live ? row : 0) * M.row_stride;
    const int ngroups = (nb + P - 1) / P;
    // producer wave pw = wave - 1 handles blocks P j + pw
    const int pw = wave - 1;
    // the scale byte (offset 16) is loaded as the top byte of the dword at
    // offset 13 and extracted where it is used: a byte load's zero-extension
    // is placed by the compiler right after the load, which waits for it
    auto load_blk = [&](int b, uint4 &q, uint32_t &e4) {
        const int bb = min(b, nb - 1);  // past the end: a clamped, unused load
        q = ld16(rp + bb * 17);
        e4 = ld4(rp + bb * 17 + 13);
    };
    // the 32 x values of one block, loaded a group ahead of their use
    struct XBlk {
        float v[32];
    };
    auto load_x = [&](int b, XBlk &xr) {
        // x is the same for every row: scalar loads (the block index is
        // wave-uniform), an SGPR operand per multiply, no LDS traffic
        const const_f32_ptr p = (const_f32_ptr)xs + min(b, nb - 1) * 32;
#pragma unroll
        for (int i = 0; i < 32; i++) xr.v[i] = p[i];
        // pin the loads here, ahead of the barrier that follows (its
        // lgkmcnt(0) covers them), instead of next to their first use
#pragma unroll
        for (int i = 0; i < 32; i++) asm volatile("" ::"s"(xr.v[i]));
    };
    auto produce = [&](int b, const uint4 &q, uint32_t e4, const XBlk &xr) {
        if (b >= nb) return;
        const uint32_t e = e4 >> 24;
        const float sc = mxfp4_scale(e);
        float *dst = &s_t[b % SLOTS][lane * 4];
        const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
        // lut[nibble] * scale is exact (two significant bits times a power of
        // two), which the hardware FP4 conversion computes for both nibbles of
        // a byte at once; a subnormal (e = 0) or infinite (e = 255) scale takes
        // the table.  The choice is made once per wave and block, so the
        // common case runs without divergent branches.
        auto store = [&](int k, const float (&t)[8]) {
            *(float4 *)(dst + 256 * (2 * k)) = make_float4(t[0], t[1], t[2], t[3]);
            *(float4 *)(dst + 256 * (2 * k + 1)) = make_float4(t[4], t[5], t[6], t[7]);
        };
        if (__builtin_amdgcn_ballot_w64(e == 0u || e == 255u) == 0) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float t[8];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const fp4x2_f32 p = fp4x2_scaled(wd[k], sc, u);
                    t[2 * u] = p.x * xr.v[8 * k + 2 * u];
                    t[2 * u + 1] = p.y * xr.v[8 * k + 2 * u + 1];
                }
                store(k, t);
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float t[8];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const uint32_t byte = (wd[k] >> (8 * u)) & 0xFFu;
                    t[2 * u] = s_lut[byte & 0xFu] * sc * xr.v[8 * k + 2 * u];
                    t[2 * u + 1] = s_lut[byte >> 4] * sc * xr.v[8 * k + 2 * u + 1];
                }
                store(k, t);
            }
        }
    };
    // MX_D groups of block loads in flight per producer: a group's worth of
    // the adder's work is far shorter than one load's latency.  Group g's
    // bytes live in ring entry g % MX_D; every index below is a constant
    // after unrolling, so the ring stays in registers.  The adder and the
    // producers run separate loops with the same barrier count (1 + npad),
    // the group count rounded up to MX_D: groups past the end add nothing,
    // produce nothing and load a clamped block, so the producer loop body is
    // straight-line and its loads retire in issue order.
    const int npad = (ngroups + MX_D - 1) / MX_D * MX_D;
    uint4 q[MX_D];
    uint32_t e[MX_D];
    if (wave > 0) {
#pragma unroll
        for (int u = 0; u < MX_D; u++) load_blk(P * u + pw, q[u], e[u]);
    }
    __syncthreads();  // the LUT staged
    if (wave == 0) {
        lds_barrier();  // group 0 produced
        float sum = 0.0f;
        // group j: the next block's eight reads are in flight while this
        // block's 32 adds run.  Every block of a full group is added without
        // a condition, so the reads stay ahead of the adds (a conditional add
        // would draw its reads into its branch, next to their use)
        auto group = [&](int j, bool full) {
            const int b0 = P * j;
            float4 v[2][8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[0][k] = *(const float4 *)(&s_t[b0 % SLOTS][lane * 4] + 256 * k);
#pragma unroll
            for (int i = 0; i < P; i++) {
                if (i + 1 < P) {
#pragma unroll
                    for (int k = 0; k < 8; k++)
                        v[(i + 1) & 1][k] = *(const float4 *)(&s_t[(b0 + i + 1) % SLOTS][lane * 4] + 256 * k);
                }
                if (full || b0 + i < nb) {
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        sum += v[i & 1][k].x;
                        sum += v[i & 1][k].y;
                        sum += v[i & 1][k].z;
                        sum += v[i & 1][k].w;
                    }
                }
                // the next block's reads stay here, one block ahead (issued
                // all at once, a group's 32 reads overrun the LDS counter)
                __builtin_amdgcn_sched_barrier(0);
            }
            lds_barrier();
        };
        int j = 0;
        for (; j + 1 < ngroups; j++) group(j, true);
        group(j, false);
        // the producers' padding groups: barriers only
        for (j++; j < npad; j++) lds_barrier();
        if (live) {
            float out = sum;
            if (bias) out += bias[row];
            if (A.epi == EPI_ADD)
                M.y[row] += out;
            else
                M.y[row] = out;
        }
        return;
    }
    XBlk xr;
    load_x(pw, xr);
    produce(pw, q[0], e[0], xr);
    load_blk(P * MX_D + pw, q[0], e[0]);
    load_x(P + pw, xr);
    lds_barrier();
    for (int j0 = 0; j0 < npad; j0 += MX_D) {
#pragma unroll
        for (int u = 0; u < MX_D; u++) {
            // group j0 + u + 1 from ring entry (u + 1) % MX_D, which then
            // takes the loads of group j0 + u + 1 + MX_D
            const int r = (u + 1) % MX_D, b = P * (j0 + u + 1) + pw;
            produce(b, q[r], e[r], xr);
            load_blk(P * (j0 + u + 1 + MX_D) + pw, q[r], e[r]);
            load_x(b + P, xr);
            lds_barrier();
        }
    }
}

// MXFP4 rows in the same order, one wave per 64-row tile that computes the
// terms and the running sums itself (lane = row).  Per block that is 16 FP4
// conversions, 32 multiplies and the 32 dependent adds on one wave: slower per
// tile than the producer/adder workgroup above, but with 64 threads per
// workgroup every SIMD holds a tile, the choice for launches with more tiles
// than CUs.  The weights arrive in chunks of 16 blocks: 64 rows x 272 bytes =
// 1088 aligned 16-byte pieces, piece f = row * 17 + p, moved by 17 coalesced
// direct global->LDS loads (instruction i carries pieces 64 i .. 64 i + 63,
// about four rows' contiguous bytes) into a 17 KB LDS chunk; each lane then
// reads its row's 272 bytes into registers (17 reads; the 17-piece row stride
// keeps them conflict-free), the next chunk's loads start, and the 17-byte
// blocks are funnel-shifted out of the registers.  A row-per-lane global load
// would touch 64 cache lines per instruction.
#define MXF_C 16  // blocks per chunk
// sum += t[i] for i = 0..3 in order, and n[i] = x[4 G + i] * p[i] issued
// between the adds, so each add's operand sum is two instructions old.  x[e]
// of the block is in row lane e % 16 of xh (the pair's half e / 16), taken by
// a DPP row broadcast.  One asm statement, so the compiler keeps the
// interleaving; the leading s_nop gives a DPP read of xh two wait states
// after any VALU write of it before the statement.
#define MX_AM4_DPP(R0, R1, R2, R3)                                                            \
    asm("s_nop 0\n\t"                                                                          \
        "v_add_f32 %0, %0, %5\n\t"                                                             \
        "v_mul_f32_dpp %1, %9, %10 row_newbcast:" #R0 " row_mask:0xf bank_mask:0xf\n\t"       \
        "v_add_f32 %0, %0, %6\n\t"                                                             \
        "v_mul_f32_dpp %2, %9, %11 row_newbcast:" #R1 " row_mask:0xf bank_mask:0xf\n\t"       \
        "v_add_f32 %0, %0, %7\n\t"                                                             \
        "v_mul_f32_dpp %3, %9, %12 row_newbcast:" #R2 " row_mask:0xf bank_mask:0xf\n\t"       \
        "v_add_f32 %0, %0, %8\n\t"                                                             \
        "v_mul_f32_dpp %4, %9, %13 row_newbcast:" #R3 " row_mask:0xf bank_mask:0xf"           \
        : "+v"(sum), "=&v"(n[0]), "=&v"(n[1]), "=&v"(n[2]), "=&v"(n[3])                         \
        : "v"(t[0]), "v"(t[1]), "v"(t[2]), "v"(t[3]), "v"(xh), "v"(p[0]), "v"(p[1]), "v"(p[2]), \
          "v"(p[3]))
template <int G>
__device__ __forceinline__ void mx_add4_mul4_dpp(float &sum, const float *t, float xh, const float *p, float *n) {
    if constexpr ((G & 3) == 0)
        MX_AM4_DPP(0, 1, 2, 3);
    else if constexpr ((G & 3) == 1)
        MX_AM4_DPP(4, 5, 6, 7);
    else if constexpr ((G & 3) == 2)
        MX_AM4_DPP(8, 9, 10, 11);
    else
        MX_AM4_DPP(12, 13, 14, 15);
}
#undef MX_AM4_DPP
__device__ __forceinline__ float swiglu_gpt_oss_ref(float g, float u);
__device__ __forceinline__ int moe_topk_wave(const float *logits, int n, int k, int slot, int32_t *sel, float *prob);

// SWI = false: tile t is 64 rows of one matrix, lane = row.  SWI = true (the
// routed experts' gate/up with gpt-oss's SwiGLU as the epilogue): matrices
// 0..n/2-1 are the gates and n/2.. the ups of the same experts; tile t is 32
// rows of gate matrix g (lanes 0..31) and the same 32 rows of up matrix g +
// n/2 (lanes 32..63), each lane's row summed exactly as without SWI, its
// bias added, then lane l < 32 stores swiglu_gpt_oss(gate, up of lane l + 32)
// at the gate's row, as moe_swiglu_kernel would from the two stored rows.
template <bool SWI>
__global__ __launch_bounds__(64) void gemv_mxfp4_fused_kernel(GemvArgs A) {
    __shared__ __align__(16) uint4 s_b[64 * 17];
    // x, K floats rounded up to 256, each 32-element block stored as 16
    // pairs (x[i], x[i + 16]): lane l reads its pair for element row l % 16
    extern __shared__ __align__(16) float s_x[];
    const int K = A.K, nb = K >> 5, lane = threadIdx.x;
    const int tile = blockIdx.x;
    const int n_sel = SWI ? A.n_mats / 2 : A.n_mats;  // matrices the tiles are counted over
    int mi = 0;
#pragma unroll
    for (int t = 1; t < GEMV_MAX_MATS; t++)
        if (t < n_sel && tile >= A.m[t].tile_begin) mi = t;
    const GemvMat M = mat_sel(A, mi);
    const GemvMat MU = SWI ? mat_sel(A, mi + n_sel) : M;  // SWI: the up matrix of the same expert
    const float *xs = M.x ? M.x : A.x;
    // x into LDS (loads in flight during the expert selection, stores after
    // it): every block then takes its x with one LDS read of a fixed latency,
    // where scalar loads would wait behind the weight stream.  Ordinary loads
    // and stores, not direct loads: LDS filled by direct loads makes the
    // compiler wait for every outstanding direct load before each read of it.
    constexpr int XQ = 12;  // 16-byte pieces per lane and batch (K <= 3072 in one)
    const int k4 = K / 4;
    float4 xv[XQ];
    auto x_load = [&](int base) {
#pragma unroll
        for (int i = 0; i < XQ; i++) xv[i] = ((const float4 *)xs)[min(base + 64 * i + lane, k4 - 1)];
    };
    // piece q holds x[4 q .. 4 q + 3]: one half (4 q & 16) of block 4 q / 32,
    // element rows r .. r + 3 (r = 4 q & 15), stored at 32 b + 2 r + h
    auto x_store = [&](int base) {
#pragma unroll
        for (int i = 0; i < XQ; i++) {
            const int q = base + 64 * i + lane;
            if (q < k4) {
                float *d = &s_x[(4 * q & ~31) + 2 * (4 * q & 15) + ((4 * q >> 4) & 1)];
                d[0] = xv[i].x;
                d[2] = xv[i].y;
                d[4] = xv[i].z;
                d[6] = xv[i].w;
            }
        }
    };
    x_load(0);
    const uint8_t *w = M.w, *wu = MU.w;
    const float *bias = M.bias, *bias_u = MU.bias;
    if (M.sel) {
        const int64_t e = A.topk_logits
                              ? moe_topk_wave(A.topk_logits, A.topk_n, A.topk_k, (int)(M.sel - A.topk_sel),
                                              blockIdx.x == 0 ? A.topk_sel : nullptr, A.topk_prob)
                              : *M.sel;
        w += e * M.sel_w;
        wu += e * MU.sel_w;
        if (bias) bias += e * M.sel_b;
        if (bias_u) bias_u += e * MU.sel_b;
    }
    x_store(0);
    for (int base = 64 * XQ; base < k4; base += 64 * XQ) {
        x_load(base);
        x_store(base);
    }
    constexpr int TR = SWI ? 32 : 64;  // rows of one matrix per tile
    const bool up_lane = SWI && lane >= 32;
    const int row0 = (tile - M.tile_begin) * TR, row = row0 + (SWI ? (lane & 31) : lane);
    const bool live = row < M.rows;
    const int64_t stride = M.row_stride;  // a multiple of 16 that holds nb * 17 bytes (the same for the ups)
    const int nch = (nb + MXF_C - 1) / MXF_C;
    // the 17 pieces this lane moves per chunk: piece f = 64 i + lane of the
    // tile is tile row f / 17, bytes 16 (f % 17) of the chunk (SWI: tile rows
    // 32.. are the up matrix's); rows past the matrix read its last row and
    // bytes past the row's end its last piece
    auto issue_chunk = [&](int c) {
        int r = lane / 17, p = lane - 17 * (lane / 17);
#pragma unroll
        for (int i = 0; i < 17; i++) {
            const bool ru = SWI && r >= 32;
            const int rr = min(row0 + (SWI ? (r & 31) : r), M.rows - 1);
            const int64_t off = min((int64_t)(MXF_C * 17 * c + 16 * p), stride - 16);
            dma16((ru ? wu : w) + (int64_t)rr * stride + off, &s_b[64 * i]);
            r += 3;  // 64 = 3 * 17 + 13
            p += 13;
            if (p >= 17) {
                p -= 17;
                r += 1;
            }
        }
    };
    struct XBlk {
        float v[32];
    };
    // block b's x as 32 uniform values (broadcast LDS reads), for the terms
    // computed outside the pipelined adds
    auto load_x = [&](int b, XBlk &xr) {
        const float *p = &s_x[min(b, nb - 1) * 32];
#pragma unroll
        for (int i = 0; i < 32; i++) xr.v[i] = p[2 * (i & 15) + (i >> 4)];
    };
    // block b's x pair of this lane: (x[32 b + l % 16], x[32 b + 16 + l % 16])
    auto load_xp = [&](int b) { return *(const float2 *)&s_x[min(b, nb - 1) * 32 + 2 * (lane & 15)]; };
    // one block's 32 terms (lut[n] * scale) * x in element order.  fast: the
    // hardware conversion gives lut * scale exactly when the lane's scale is
    // normal; table: any scale byte (0 is the subnormal 2^-127, 255 infinite)
    auto terms_fast = [&](const uint32_t (&wd)[4], uint32_t e, const XBlk &xr, float (&t)[32]) {
        const float sc = mxfp4_scale(e);
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const fp4x2_f32 p = fp4x2_scaled(wd[k], sc, u);
                t[8 * k + 2 * u] = p.x * xr.v[8 * k + 2 * u];
                t[8 * k + 2 * u + 1] = p.y * xr.v[8 * k + 2 * u + 1];
            }
    };
    auto terms_table = [&](const uint32_t (&wd)[4], uint32_t e, const XBlk &xr, float (&t)[32]) {
        const float sc = mxfp4_scale(e);
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int u = 0; u < 4; u++) {
                // lut[n] itself from the conversion at scale 1, then the
                // reference's (lut * scale) * x
                const fp4x2_f32 q = fp4x2_scaled(wd[k], 1.0f, u);
                t[8 * k + 2 * u] = q.x * sc * xr.v[8 * k + 2 * u];
                t[8 * k + 2 * u + 1] = q.y * sc * xr.v[8 * k + 2 * u + 1];
            }
    };
    // e == 0 or e == 255 in one unsigned compare
    auto rare_scale = [](uint32_t e) { return __builtin_amdgcn_ballot_w64(e - 1u > 253u) != 0; };
    // block j of this lane's chunk: bytes 17 j .. 17 j + 16 of the 68 dwords
    auto block_of = [&](const uint32_t (&dw)[68], int j, uint32_t (&wd)[4], uint32_t &e) {
        const int d = (17 * j) >> 2, o = (17 * j) & 3;
#pragma unroll
        for (int k = 0; k < 4; k++) wd[k] = o ? __builtin_amdgcn_alignbyte(dw[d + k + 1], dw[d + k], o) : dw[d + k];
        e = (dw[d + 4] >> (8 * o)) & 0xFFu;
    };
    // The running sum is a chain of dependent adds; the terms are not.  Block
    // j's 32 adds alternate with the multiplies of block j + 1's terms, whose
    // x enters each multiply through a DPP row broadcast of the lane's x pair
    // (mx_add4_mul4_dpp), so each add finds its predecessor's result ready.
    // T[j & 1] holds block j's terms, XP[b & 1] block b's x pair, read a
    // block before the block whose adds it joins.
    float sum = 0.0f;
    float2 XP[2];
    XP[1] = load_xp(1);
    issue_chunk(0);
    for (int c = 0; c < nch; c++) {
        // chunk c (and, before the first, x): from LDS into registers, then
        // chunk c + 1 into the freed LDS while this one is summed
        RH_WAIT_VM(0);
        uint32_t dw[68];
        const uint4 *src = &s_b[17 * lane];
#pragma unroll
        for (int p = 0; p < 17; p++) {
            const uint4 v = src[p];
            dw[4 * p] = v.x;
            dw[4 * p + 1] = v.y;
            dw[4 * p + 2] = v.z;
            dw[4 * p + 3] = v.w;
        }
        RH_WAIT_LGKM0();
        if (c + 1 < nch) issue_chunk(c + 1);  // uniform
        const int b0 = MXF_C * c;
        XP[0] = load_xp(b0 + 2);
        float T[2][32];
        {
            XBlk xr;
            load_x(b0, xr);
            uint32_t wd[4], e;
            block_of(dw, 0, wd, e);
            if (rare_scale(e))
                terms_table(wd, e, xr, T[0]);
            else
                terms_fast(wd, e, xr, T[0]);
        }
#pragma unroll
        for (int j = 0; j < MXF_C; j++) {
            if (b0 + j < nb) {  // uniform; false only in a last, partial chunk
                const float(&t)[32] = T[j & 1];
                if (j + 1 < MXF_C) {
                    // block j + 1's terms between block j's adds (past the
                    // row's end: values that are never added)
                    float(&tn)[32] = T[(j + 1) & 1];
                    const float2 xp = XP[(j + 1) & 1];
                    uint32_t wd[4], e;
                    block_of(dw, j + 1, wd, e);
                    // 2^(e-127) for a normal scale byte; the others take the
                    // table form below, whatever this gives them
                    const float sc = __builtin_bit_cast(float, e << 23);
                    float pr[32];
#pragma unroll
                    for (int k = 0; k < 4; k++)
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            const fp4x2_f32 q = fp4x2_scaled(wd[k], sc, u);
                            pr[8 * k + 2 * u] = q.x;
                            pr[8 * k + 2 * u + 1] = q.y;
                        }
                    mx_add4_mul4_dpp<0>(sum, &t[0], xp.x, &pr[0], &tn[0]);
                    mx_add4_mul4_dpp<1>(sum, &t[4], xp.x, &pr[4], &tn[4]);
                    mx_add4_mul4_dpp<2>(sum, &t[8], xp.x, &pr[8], &tn[8]);
                    mx_add4_mul4_dpp<3>(sum, &t[12], xp.x, &pr[12], &tn[12]);
                    mx_add4_mul4_dpp<4>(sum, &t[16], xp.y, &pr[16], &tn[16]);
                    mx_add4_mul4_dpp<5>(sum, &t[20], xp.y, &pr[20], &tn[20]);
                    mx_add4_mul4_dpp<6>(sum, &t[24], xp.y, &pr[24], &tn[24]);
                    mx_add4_mul4_dpp<7>(sum, &t[28], xp.y, &pr[28], &tn[28]);
                    if (rare_scale(e)) {
                        XBlk xr;
                        load_x(b0 + j + 1, xr);
                        terms_table(wd, e, xr, tn);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 32; i++) sum += t[i];
                }
                if (j + 1 < MXF_C) XP[(j + 1) & 1] = load_xp(b0 + j + 3);  // block j + 1's pair is no longer needed
            }
        }
    }
    if constexpr (SWI) {
        const float *bl = up_lane ? bias_u : bias;
        float out = sum;
        if (bl && live) out += bl[row];
        const float u = __shfl_down(out, 32);  // lane l < 32: the up row's value from lane l + 32
        if (!up_lane && live) M.y[row] = swiglu_gpt_oss_ref(out, u);
    } else if (live) {
        float out = sum;
        if (bias) out += bias[row];
        if (A.epi == EPI_ADD)
            M.y[row] += out;
        else
            M.y[row] = out;
    }
}

// ---- debug kernels: per-block integer parts (bit-exactness checks) -----------
// Q4_K: out[row*nb*2 + 2b] = isum, +1 = imin.  Q6_K: out[row*nb + b] = isum.
// Q8_0: out[row*nb32 + b] = s (int dot of the 32-block).
__global__ void block_ints_kernel(const uint8_t *w, int64_t row_stride, int rows, int K, int fmt, XQ xq, int *out) {
    int row = blockIdx.x;
    if (row >= rows) return;
    const uint8_t *wr = w + (int64_t)row * row_stride;
    if (fmt == F_Q8_0) {
        int nb = K >> 5;
        for (int b = threadIdx.x; b < nb; b += blockDim.x) {
            const uint8_t *blk = wr + b * 34;
            uint4 a = ld16(blk + 2), c = ld16(blk + 18);
            const int32_t *x = (const int32_t *)(xq.qs + b * 32);
            int s = 0;
            s = sdot4(a.x, x[0], s); s = sdot4(a.y, x[1], s); s = sdot4(a.z, x[2], s); s = sdot4(a.w, x[3], s);
            s = sdot4(c.x, x[4], s); s = sdot4(c.y, x[5], s); s = sdot4(c.z, x[6], s); s = sdot4(c.w, x[7], s);
            out[(int64_t)row * nb + b] = s;
        }
        return;
    }
    int nb = K >> 8;
    for (int b = threadIdx.x; b < nb; b += blockDim.x) {
        const int32_t *xq32 = (const int32_t *)(xq.qs + b * 256);
        if (fmt == F_Q4_K) {
            int isum = 0, imin = 0;
            for (int q = 0; q < 4; q++) {
                Q4KLoad L = q4k_load(wr + b * 144, q);
                int a, m;
                q4k_unit(L, q, q4k_scale_sel(q), xq32, xq.bsums + b * 8, a, m);
                isum += a;
                imin += m;
            }
            out[((int64_t)row * nb + b) * 2] = isum;
            out[((int64_t)row * nb + b) * 2 + 1] = imin;
        } else {
            int isum = 0;
            for (int q = 0; q < 4; q++) {
                Q6KLoad L = q6k_load(wr + b * 210, q);
                isum += q6k_unit(L, q, xq32, xq.sums16 + b * 16);
            }
            out[(int64_t)row * nb + b] = isum;
        }
    }
}

// ---- dequantization (bit-exact with src/simd.rs:4044-4294) --------------------
__global__ void dequant_rows_kernel(const uint8_t *w, int64_t row_stride, int rows, int K, int fmt, float *out) {
    int row = blockIdx.y;
    if (row >= rows) return;
    const uint8_t *wr = w + (int64_t)row * row_stride;
    float *o = out + (int64_t)row * K;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < K; e += gridDim.x * blockDim.x) {
        float v = 0.0f;
        if (fmt == F_Q8_0) {
            const uint8_t *blk = wr + (e >> 5) * 34;
            v = ldh(blk) * (float)(int8_t)blk[2 + (e & 31)];
        } else if (fmt == F_Q4_K) {
            const uint8_t *blk = wr + (e >> 8) * 144;
            int p = e & 255, j = p >> 6, hi = (p >> 5) & 1, l = p & 31;
            uint32_t s03 = ld4(blk + 4), s47 = ld4(blk + 8), s811 = ld4(blk + 12);
            int sc, m;
            scale_min_k4(2 * j + hi, s03, s47, s811, sc, m);
            float d1 = ldh(blk) * (float)sc, m1 = ldh(blk + 2) * (float)m;
            uint8_t byte = blk[16 + 32 * j + l];
            int qv = hi ? (byte >> 4) : (byte & 0xF);
            v = d1 * (float)qv - m1;
        } else if (fmt == F_Q6_K) {
            const uint8_t *blk = wr + (e >> 8) * 210;
            int p = e & 255, n = p >> 7, pp = p & 127, k = pp >> 5, l = pp & 31;
            const uint8_t *ql = blk + 64 * n, *qh = blk + 128 + 32 * n;
            const int8_t *sc = (const int8_t *)(blk + 192 + 8 * n);
            uint8_t lo = (k & 1) ? ql[l + 32] : ql[l];
            int nib = (k & 2) ? (lo >> 4) : (lo & 0xF);
            int q = (nib | (((qh[l] >> (2 * k)) & 3) << 4)) - 32;
            v = ldh(blk + 208) * (float)sc[l / 16 + 2 * k] * (float)q;
        } else if (fmt == F_MXFP4) {
            const uint8_t *blk = wr + (e >> 5) * 17;
            int p = e & 31;
            uint8_t byte = blk[p >> 1];
            v = kMxfp4Lut[(p & 1) ? (byte >> 4) : (byte & 0xF)] * mxfp4_scale(blk[16]);
        }
        o[e] = v;
    }
}

}  // namespace rh
