/*
 * oracle.c — CPU restatement of RustyLLM's x86-64 decode-step numerics.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  It is the checker the HIP path is
 * compared against and the CPU baseline bench.py reports; it never runs on the
 * product path.
 *
 * Citations are to SimonWaldherr/RustyLLM: "simd.rs:N" means src/simd.rs line
 * N, "model.rs:N" means src/model.rs line N, and so on.  The AVX2 functions use
 * the same intrinsic sequence as the reference so lane assignment and rounding
 * points match; the build uses -ffp-contract=off so no other FMA appears.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* f16 -> f32, simd.rs:2011-2036 (f16_to_f32_soft; the LUT of simd.rs:485-494
 * stores exactly these values).                                              */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            uint32_t e = 0, m = mant;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                e += 1;
            }
            m &= 0x3ffu;
            uint32_t ee = 127 - 15 + 1 - e;
            bits = (sign << 31) | (ee << 23) | (m << 13);
        }
    } else if (exp == 31) {
        bits = (sign << 31) | (0xffu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float f16le(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* MXFP4 helpers, simd.rs:5851-5882.  2.0f32.powi(e-127) is an exact power of
 * two (2^-127 is a representable subnormal, 2^128 overflows to inf), which is
 * what ldexpf returns.                                                         */
static const float MXFP4_LUT[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
float orc_mxfp4_scale(uint8_t e) { return ldexpf(1.0f, (int)e - 127); }

/* get_scale_min_k4, simd.rs:4537-4546 */
static inline void get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ------------------------------------------------------------------------ */
/* Q8_K quantizer, scalar: simd.rs:5013-5033                                 */
void orc_quantize_row_q8k_scalar(const float *x, int64_t n, int8_t *qs, float *d, int16_t *bsums) {
    int64_t nb = n / 256;
    for (int64_t b = 0; b < nb; b++) {
        const float *xb = x + b * 256;
        float amax = 0.0f;
        for (int i = 0; i < 256; i++) amax = fmaxf(amax, fabsf(xb[i]));
        d[b] = amax * (1.0f / 127.0f);
        float id = amax > 0.0f ? 127.0f / amax : 0.0f;
        for (int sub = 0; sub < 8; sub++) {
            int32_t sum = 0;
            for (int l = 0; l < 32; l++) {
                float v = nearbyintf(xb[sub * 32 + l] * id); /* ties-to-even (default mode) */
                int32_t q = isnan(v) ? 0 : (v > 2147483520.0f ? INT32_MAX : (v < -2147483648.0f ? INT32_MIN : (int32_t)v));
                if (q < -128) q = -128;
                if (q > 127) q = 127;
                qs[b * 256 + sub * 32 + l] = (int8_t)q;
                sum += q;
            }
            bsums[b * 8 + sub] = (int16_t)sum;
        }
    }
}

/* Q8_K quantizer, AVX2: simd.rs:5050-5101                                   */
__attribute__((target("avx2,fma")))
void orc_quantize_row_q8k_avx2(const float *x, int64_t n, int8_t *qs, float *d, int16_t *bsums) {
    int64_t nb = n / 256;
    const __m256 sign_mask = _mm256_set1_ps(-0.0f);
    const __m256i perm = _mm256_setr_epi32(0, 4, 1, 5, 2, 6, 3, 7);
    for (int64_t b = 0; b < nb; b++) {
        const float *xb = x + b * 256;
        __m256 amax_v = _mm256_setzero_ps();
        for (int i = 0; i < 32; i++) {
            __m256 v = _mm256_loadu_ps(xb + i * 8);
            amax_v = _mm256_max_ps(amax_v, _mm256_andnot_ps(sign_mask, v));
        }
        __m128 hi = _mm256_extractf128_ps(amax_v, 1);
        __m128 m4 = _mm_max_ps(_mm256_castps256_ps128(amax_v), hi);
        __m128 m2 = _mm_max_ps(m4, _mm_movehl_ps(m4, m4));
        __m128 m1 = _mm_max_ss(m2, _mm_shuffle_ps(m2, m2, 0x55));
        float amax = _mm_cvtss_f32(m1);
        d[b] = amax * (1.0f / 127.0f);
        float id = amax > 0.0f ? 127.0f / amax : 0.0f;
        __m256 idv = _mm256_set1_ps(id);
        int8_t *qb = qs + b * 256;
        for (int sub = 0; sub < 8; sub++) {
            int off = sub * 32;
            __m256i i0 = _mm256_cvtps_epi32(_mm256_mul_ps(_mm256_loadu_ps(xb + off), idv));
            __m256i i1 = _mm256_cvtps_epi32(_mm256_mul_ps(_mm256_loadu_ps(xb + off + 8), idv));
            __m256i i2 = _mm256_cvtps_epi32(_mm256_mul_ps(_mm256_loadu_ps(xb + off + 16), idv));
            __m256i i3 = _mm256_cvtps_epi32(_mm256_mul_ps(_mm256_loadu_ps(xb + off + 24), idv));
            __m256i sum_v = _mm256_add_epi32(_mm256_add_epi32(i0, i1), _mm256_add_epi32(i2, i3));
            __m128i sum_hi = _mm256_extracti128_si256(sum_v, 1);
            __m128i s4 = _mm_add_epi32(_mm256_castsi256_si128(sum_v), sum_hi);
            __m128i s2 = _mm_add_epi32(s4, _mm_unpackhi_epi64(s4, s4));
            __m128i s1 = _mm_add_epi32(s2, _mm_shuffle_epi32(s2, 0x55));
            bsums[b * 8 + sub] = (int16_t)_mm_cvtsi128_si32(s1);
            __m256i p01 = _mm256_packs_epi32(i0, i1);
            __m256i p23 = _mm256_packs_epi32(i2, i3);
            __m256i packed = _mm256_packs_epi16(p01, p23);
            __m256i ordered = _mm256_permutevar8x32_epi32(packed, perm);
            _mm256_storeu_si256((__m256i *)(qb + off), ordered);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* dequantization: simd.rs:4044-4055 (Q8_0), 4162-4196 (Q4_K), 4244-4276
 * (Q6_K), 4280-4294 (MXFP4).  Tail past whole blocks is zero-filled
 * (clear_dequant_tail, simd.rs:4037-4042).                                   */
static void dequant_q8_0(const uint8_t *q, float *out, int64_t n) {
    int64_t nb = n / 32;
    for (int64_t i = nb * 32; i < n; i++) out[i] = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = q + b * 34;
        float scale = f16le(blk);
        for (int i = 0; i < 32; i++) out[b * 32 + i] = scale * (float)(int8_t)blk[2 + i];
    }
}

static void dequant_q4_k(const uint8_t *qrow, float *out, int64_t n) {
    int64_t nb = n / 256;
    for (int64_t i = nb * 256; i < n; i++) out[i] = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = qrow + b * 144;
        float d = f16le(blk), dmin = f16le(blk + 2);
        const uint8_t *scales = blk + 4;
        const uint8_t *q = blk + 16;
        int is = 0;
        for (int j = 0; j < 256; j += 64) {
            uint8_t sc1, m1, sc2, m2;
            get_scale_min_k4(is, scales, &sc1, &m1);
            float d1 = d * (float)sc1, min1 = dmin * (float)m1;
            get_scale_min_k4(is + 1, scales, &sc2, &m2);
            float d2 = d * (float)sc2, min2 = dmin * (float)m2;
            for (int l = 0; l < 32; l++) out[b * 256 + j + l] = d1 * (float)(q[l] & 0x0F) - min1;
            for (int l = 0; l < 32; l++) out[b * 256 + j + 32 + l] = d2 * (float)(q[l] >> 4) - min2;
            q += 32;
            is += 2;
        }
    }
}

static void dequant_q6_k(const uint8_t *qrow, float *out, int64_t n) {
    int64_t nb = n / 256;
    for (int64_t i = nb * 256; i < n; i++) out[i] = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = qrow + b * 210;
        const uint8_t *ql = blk, *qh = blk + 128;
        const int8_t *sc = (const int8_t *)(blk + 192);
        float d = f16le(blk + 208);
        float *y = out + b * 256;
        for (int nn = 0; nn < 256; nn += 128) {
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                float q1 = (float)((int)((ql[l] & 0x0F) | ((qh[l] & 0x03) << 4)) - 32);
                float q2 = (float)((int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 0x03) << 4)) - 32);
                float q3 = (float)((int)((ql[l] >> 4) | (((qh[l] >> 4) & 0x03) << 4)) - 32);
                float q4 = (float)((int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 0x03) << 4)) - 32);
                y[nn + l] = d * (float)sc[is] * q1;
                y[nn + 32 + l] = d * (float)sc[is + 2] * q2;
                y[nn + 64 + l] = d * (float)sc[is + 4] * q3;
                y[nn + 96 + l] = d * (float)sc[is + 6] * q4;
            }
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

static void dequant_mxfp4(const uint8_t *qrow, float *out, int64_t n) {
    int64_t nb = n / 32;
    for (int64_t i = nb * 32; i < n; i++) out[i] = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = qrow + b * 17;
        float scale = orc_mxfp4_scale(blk[16]);
        for (int i = 0; i < 16; i++) {
            uint8_t byte = blk[i];
            out[b * 32 + i * 2] = MXFP4_LUT[byte & 0x0F] * scale;
            out[b * 32 + i * 2 + 1] = MXFP4_LUT[byte >> 4] * scale;
        }
    }
}

void orc_dequant_row(int dtype, const uint8_t *q, float *out, int64_t n) {
    switch (dtype) {
    case ORC_F32: memcpy(out, q, (size_t)n * 4); break;
    case ORC_Q8_0: dequant_q8_0(q, out, n); break;
    case ORC_Q4_K: dequant_q4_k(q, out, n); break;
    case ORC_Q6_K: dequant_q6_k(q, out, n); break;
    case ORC_MXFP4: dequant_mxfp4(q, out, n); break;
    default: memset(out, 0, (size_t)n * 4); break;
    }
}

/* ------------------------------------------------------------------------ */
/* horizontal sums: simd.rs:6534-6545 (hsum_avx), 6724-6732 (hsum_i32_avx2)   */
__attribute__((target("avx2,fma")))
static inline float hsum_avx(__m256 v) {
    __m128 lo = _mm256_extractf128_ps(v, 0);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 sum4 = _mm_add_ps(lo, hi);
    __m128 sum2 = _mm_hadd_ps(sum4, sum4);
    __m128 sum1 = _mm_hadd_ps(sum2, sum2);
    return _mm_cvtss_f32(sum1);
}

__attribute__((target("avx2,fma")))
static inline int32_t hsum_i32_avx2(__m256i v) {
    __m128i hi = _mm256_extracti128_si256(v, 1);
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), hi);
    s = _mm_add_epi32(s, _mm_unpackhi_epi64(s, s));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x55));
    return _mm_cvtsi128_si32(s);
}

/* dot_f32_avx2, simd.rs:6547-6586 */
__attribute__((target("avx2,fma")))
float orc_dot_f32_avx2(const float *a, const float *b, int64_t n) {
    int64_t main_ = n / 32;
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    __m256 acc2 = _mm256_setzero_ps(), acc3 = _mm256_setzero_ps();
    const float *ap = a, *bp = b;
    for (int64_t i = 0; i < main_; i++) {
        acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(ap), _mm256_loadu_ps(bp), acc0);
        acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(ap + 8), _mm256_loadu_ps(bp + 8), acc1);
        acc2 = _mm256_fmadd_ps(_mm256_loadu_ps(ap + 16), _mm256_loadu_ps(bp + 16), acc2);
        acc3 = _mm256_fmadd_ps(_mm256_loadu_ps(ap + 24), _mm256_loadu_ps(bp + 24), acc3);
        ap += 32;
        bp += 32;
    }
    __m256 acc = _mm256_add_ps(_mm256_add_ps(acc0, acc1), _mm256_add_ps(acc2, acc3));
    int64_t tail_start = main_ * 32;
    int64_t tail_8 = (n - tail_start) / 8;
    for (int64_t i = 0; i < tail_8; i++) {
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(ap), _mm256_loadu_ps(bp), acc);
        ap += 8;
        bp += 8;
    }
    float sum = hsum_avx(acc);
    for (int64_t i = tail_start + tail_8 * 8; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* dot_f32x4_avx2, simd.rs:6588-6619 */
__attribute__((target("avx2,fma")))
static void dot_f32x4_avx2(const float *a0, const float *a1, const float *a2, const float *a3,
                           const float *b, int64_t n, float out[4]) {
    __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
    __m256 s2 = _mm256_setzero_ps(), s3 = _mm256_setzero_ps();
    int64_t i = 0;
    while (i + 8 <= n) {
        __m256 key = _mm256_loadu_ps(b + i);
        s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a0 + i), key, s0);
        s1 = _mm256_fmadd_ps(_mm256_loadu_ps(a1 + i), key, s1);
        s2 = _mm256_fmadd_ps(_mm256_loadu_ps(a2 + i), key, s2);
        s3 = _mm256_fmadd_ps(_mm256_loadu_ps(a3 + i), key, s3);
        i += 8;
    }
    out[0] = hsum_avx(s0);
    out[1] = hsum_avx(s1);
    out[2] = hsum_avx(s2);
    out[3] = hsum_avx(s3);
    while (i < n) {
        float key = b[i];
        out[0] += a0[i] * key;
        out[1] += a1[i] * key;
        out[2] += a2[i] * key;
        out[3] += a3[i] * key;
        i++;
    }
}

/* affine_add_f32x4_avx2, simd.rs:6621-6669 */
__attribute__((target("avx2,fma")))
static void affine_add_f32x4_avx2(float *o0, float *o1, float *o2, float *o3,
                                  const float mul[4], const float alpha[4], const float *x, int64_t n) {
    float *outs[4] = {o0, o1, o2, o3};
    __m256 mv[4], av[4];
    for (int g = 0; g < 4; g++) {
        mv[g] = _mm256_set1_ps(mul[g]);
        av[g] = _mm256_set1_ps(alpha[g]);
    }
    int64_t i = 0;
    while (i + 8 <= n) {
        __m256 value = _mm256_loadu_ps(x + i);
        for (int g = 0; g < 4; g++) {
            __m256 old = _mm256_loadu_ps(outs[g] + i);
            _mm256_storeu_ps(outs[g] + i, _mm256_fmadd_ps(value, av[g], _mm256_mul_ps(old, mv[g])));
        }
        i += 8;
    }
    while (i < n) {
        for (int g = 0; g < 4; g++) outs[g][i] = outs[g][i] * mul[g] + alpha[g] * x[i];
        i++;
    }
}

/* axpy / scale / scale_add, simd.rs:7212-7272 */
__attribute__((target("avx2,fma")))
static void axpy_f32_avx2(float *out, float alpha, const float *x, int64_t n) {
    int64_t main_ = n / 8;
    __m256 av = _mm256_set1_ps(alpha);
    for (int64_t i = 0; i < main_; i++) {
        __m256 o = _mm256_loadu_ps(out + i * 8);
        _mm256_storeu_ps(out + i * 8, _mm256_fmadd_ps(av, _mm256_loadu_ps(x + i * 8), o));
    }
    for (int64_t i = main_ * 8; i < n; i++) out[i] += alpha * x[i];
}

__attribute__((target("avx2,fma")))
static void scale_f32_avx2(float *out, float scale, int64_t n) {
    int64_t main_ = n / 8;
    __m256 sv = _mm256_set1_ps(scale);
    for (int64_t i = 0; i < main_; i++) _mm256_storeu_ps(out + i * 8, _mm256_mul_ps(_mm256_loadu_ps(out + i * 8), sv));
    for (int64_t i = main_ * 8; i < n; i++) out[i] *= scale;
}

__attribute__((target("avx2,fma")))
static void scale_add_f32_avx2(float *out, float scale, const float *add, int64_t n) {
    int64_t main_ = n / 8;
    __m256 sv = _mm256_set1_ps(scale);
    for (int64_t i = 0; i < main_; i++) {
        __m256 o = _mm256_loadu_ps(out + i * 8);
        _mm256_storeu_ps(out + i * 8, _mm256_fmadd_ps(o, sv, _mm256_loadu_ps(add + i * 8)));
    }
    for (int64_t i = main_ * 8; i < n; i++) out[i] = out[i] * scale + add[i];
}

/* ------------------------------------------------------------------------ */
/* dot_q8_0_f32_avx2, simd.rs:6671-6692 */
__attribute__((target("avx2,fma")))
float orc_dot_q8_0_f32_avx2(const uint8_t *w, const float *x, int64_t n) {
    int64_t nb = n / 32;
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + b * 34;
        __m256 sv = _mm256_set1_ps(f16le(blk));
        const int8_t *qp = (const int8_t *)(blk + 2);
        const float *xp = x + b * 32;
        for (int i = 0; i < 4; i++) {
            __m128i qi128 = _mm_loadl_epi64((const __m128i *)(qp + i * 8));
            __m256 qf = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(qi128));
            acc = _mm256_fmadd_ps(_mm256_mul_ps(sv, qf), _mm256_loadu_ps(xp + i * 8), acc);
        }
    }
    return hsum_avx(acc);
}

/* dot_mxfp4_f32_scalar, simd.rs:5886-5902 (the x86 dispatch of dot_mxfp4_f32,
 * simd.rs:2752-2762, always lands here). */
float orc_dot_mxfp4_f32_scalar(const uint8_t *w, const float *x, int64_t n) {
    int64_t nb = n / 32;
    float sum = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + b * 17;
        float scale = orc_mxfp4_scale(blk[16]);
        for (int i = 0; i < 16; i++) {
            uint8_t byte = blk[i];
            sum += MXFP4_LUT[byte & 0x0F] * scale * x[b * 32 + i * 2];
            sum += MXFP4_LUT[byte >> 4] * scale * x[b * 32 + i * 2 + 1];
        }
    }
    return sum;
}

/* dot_q4_k_q8k_avx2, simd.rs:6738-6801 */
__attribute__((target("avx2,fma")))
float orc_dot_q4_k_q8k_avx2(const uint8_t *w, const int8_t *qs, const float *dxs, const int16_t *bsums, int64_t n) {
    int64_t nb = n / 256;
    const __m256i lowmask = _mm256_set1_epi8(0x0F);
    float acc = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + b * 144;
        float d = f16le(blk), dmin = f16le(blk + 2);
        const uint8_t *scales = blk + 4;
        const uint8_t *q = blk + 16;
        float dx = dxs[b];
        const int8_t *xqb = qs + b * 256;
        const int16_t *bsb = bsums + b * 8;
        __m256i isum_v = _mm256_setzero_si256();
        int32_t imin = 0;
        for (int c = 0; c < 4; c++) {
            int is = c * 2;
            uint8_t sc1, m1, sc2, m2;
            get_scale_min_k4(is, scales, &sc1, &m1);
            get_scale_min_k4(is + 1, scales, &sc2, &m2);
            __m256i raw = _mm256_loadu_si256((const __m256i *)(q + c * 32));
            __m256i lo = _mm256_and_si256(raw, lowmask);
            __m256i hi = _mm256_and_si256(_mm256_srli_epi16(raw, 4), lowmask);
            __m256i x_lo = _mm256_loadu_si256((const __m256i *)(xqb + c * 64));
            __m256i x_hi = _mm256_loadu_si256((const __m256i *)(xqb + c * 64 + 32));
            __m256i p_lo = _mm256_maddubs_epi16(lo, x_lo);
            __m256i p_hi = _mm256_maddubs_epi16(hi, x_hi);
            isum_v = _mm256_add_epi32(isum_v, _mm256_madd_epi16(p_lo, _mm256_set1_epi16((int16_t)sc1)));
            isum_v = _mm256_add_epi32(isum_v, _mm256_madd_epi16(p_hi, _mm256_set1_epi16((int16_t)sc2)));
            imin += (int32_t)m1 * (int32_t)bsb[is] + (int32_t)m2 * (int32_t)bsb[is + 1];
        }
        int32_t isum = hsum_i32_avx2(isum_v);
        acc += dx * (d * (float)isum - dmin * (float)imin);
    }
    return acc;
}

/* dot_q6_k_q8k_avx2, simd.rs:6862-6922 */
__attribute__((target("avx2,fma")))
float orc_dot_q6_k_q8k_avx2(const uint8_t *w, const int8_t *qs, const float *dxs, const int16_t *bsums, int64_t n) {
    (void)bsums;
    int64_t nb = n / 256;
    const __m256i lowmask = _mm256_set1_epi8(0x0F);
    const __m256i m3 = _mm256_set1_epi8(0x03);
    const __m256i sub32 = _mm256_set1_epi8(32);
    float acc = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + b * 210;
        float d = f16le(blk + 208);
        float dx = dxs[b];
        const int8_t *xqb = qs + b * 256;
        const int8_t *sc_base = (const int8_t *)(blk + 192);
        __m256i isum_v = _mm256_setzero_si256();
        for (int g = 0; g < 2; g++) {
            __m256i ql0 = _mm256_loadu_si256((const __m256i *)(blk + g * 64));
            __m256i ql1 = _mm256_loadu_si256((const __m256i *)(blk + g * 64 + 32));
            __m256i qhv = _mm256_loadu_si256((const __m256i *)(blk + 128 + g * 32));
            const int8_t *scs = sc_base + g * 8;
            int x_base = g * 128;
            __m256i qv[4];
            qv[0] = _mm256_or_si256(_mm256_and_si256(ql0, lowmask), _mm256_slli_epi16(_mm256_and_si256(qhv, m3), 4));
            qv[1] = _mm256_or_si256(_mm256_and_si256(ql1, lowmask),
                                    _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qhv, 2), m3), 4));
            qv[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(ql0, 4), lowmask),
                                    _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qhv, 4), m3), 4));
            qv[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(ql1, 4), lowmask),
                                    _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qhv, 6), m3), 4));
            for (int idx = 0; idx < 4; idx++) {
                __m256i qsv = _mm256_sub_epi8(qv[idx], sub32);
                __m256i xv = _mm256_loadu_si256((const __m256i *)(xqb + x_base + idx * 32));
                __m256i p = _mm256_maddubs_epi16(_mm256_abs_epi8(qsv), _mm256_sign_epi8(xv, qsv));
                int16_t sc_a = scs[idx * 2], sc_b = scs[idx * 2 + 1];
                __m256i sc_v = _mm256_set_m128i(_mm_set1_epi16(sc_b), _mm_set1_epi16(sc_a));
                isum_v = _mm256_add_epi32(isum_v, _mm256_madd_epi16(p, sc_v));
            }
        }
        acc += dx * d * (float)hsum_i32_avx2(isum_v);
    }
    return acc;
}

/* dot_q8_0_q8k_avx2, simd.rs:7179-7210 */
__attribute__((target("avx2,fma")))
float orc_dot_q8_0_q8k_avx2(const uint8_t *w, const int8_t *qs, const float *dxs, const int16_t *bsums, int64_t n) {
    (void)bsums;
    int64_t n_super = n / 256;
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc = _mm256_setzero_ps();
    for (int64_t sb = 0; sb < n_super; sb++) {
        float dx = dxs[sb];
        const int8_t *xqb = qs + sb * 256;
        const uint8_t *base = w + sb * 8 * 34;
        for (int blk = 0; blk < 8; blk++) {
            const uint8_t *block = base + blk * 34;
            float scale = dx * f16le(block);
            __m256i wv = _mm256_loadu_si256((const __m256i *)(block + 2));
            __m256i xv = _mm256_loadu_si256((const __m256i *)(xqb + blk * 32));
            __m256i p = _mm256_maddubs_epi16(_mm256_abs_epi8(wv), _mm256_sign_epi8(xv, wv));
            __m256i s = _mm256_madd_epi16(p, ones);
            acc = _mm256_fmadd_ps(_mm256_set1_ps(scale), _mm256_cvtepi32_ps(s), acc);
        }
    }
    return hsum_avx(acc);
}

/* ------------------------------------------------------------------------ */
/* Scalar integer emulations, restated from the reference's own tests
 * (simd.rs:8725-8755, 8803-8831, 8864-8882).                                */
float orc_emulate_q4_k_q8k(const uint8_t *w, const int8_t *qs, const float *dxs, const int16_t *bsums, int64_t n) {
    float acc = 0.0f;
    for (int64_t b = 0; b < n / 256; b++) {
        const uint8_t *blk = w + b * 144;
        float d = f16le(blk), dmin = f16le(blk + 2);
        const uint8_t *scales = blk + 4, *q = blk + 16;
        const int8_t *xq = qs + b * 256;
        const int16_t *bs = bsums + b * 8;
        int32_t isum = 0, imin = 0;
        for (int c = 0; c < 4; c++) {
            int is = c * 2;
            uint8_t sc1, m1, sc2, m2;
            get_scale_min_k4(is, scales, &sc1, &m1);
            get_scale_min_k4(is + 1, scales, &sc2, &m2);
            int32_t qa = 0, qb = 0;
            for (int l = 0; l < 32; l++) {
                uint8_t byte = q[c * 32 + l];
                qa += (int32_t)(byte & 0xF) * xq[c * 64 + l];
                qb += (int32_t)(byte >> 4) * xq[c * 64 + 32 + l];
            }
            isum += (int32_t)sc1 * qa + (int32_t)sc2 * qb;
            imin += (int32_t)m1 * bs[is] + (int32_t)m2 * bs[is + 1];
        }
        acc += dxs[b] * (d * (float)isum - dmin * (float)imin);
    }
    return acc;
}

float orc_emulate_q6_k_q8k(const uint8_t *w, const int8_t *qs, const float *dxs, int64_t n) {
    float acc = 0.0f;
    for (int64_t b = 0; b < n / 256; b++) {
        const uint8_t *blk = w + b * 210;
        float d = f16le(blk + 208);
        const int8_t *xq = qs + b * 256;
        int32_t isum = 0;
        for (int g = 0; g < 2; g++) {
            const uint8_t *ql = blk + g * 64, *qh = blk + 128 + g * 32;
            const int8_t *scs = (const int8_t *)(blk + 192 + g * 8);
            int base = g * 128;
            for (int l = 0; l < 32; l++) {
                int32_t q0 = (int32_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
                int32_t q1 = (int32_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int32_t q2 = (int32_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int32_t q3 = (int32_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                int si = l / 16;
                isum += scs[si] * q0 * xq[base + l] + scs[si + 2] * q1 * xq[base + 32 + l] +
                        scs[si + 4] * q2 * xq[base + 64 + l] + scs[si + 6] * q3 * xq[base + 96 + l];
            }
        }
        acc += dxs[b] * d * (float)isum;
    }
    return acc;
}

float orc_emulate_q8_0_q8k(const uint8_t *w, const int8_t *qs, const float *dxs, int64_t n) {
    float acc = 0.0f;
    for (int64_t sb = 0; sb < n / 256; sb++) {
        const int8_t *xq = qs + sb * 256;
        float inner = 0.0f;
        for (int blk = 0; blk < 8; blk++) {
            const uint8_t *block = w + (sb * 8 + blk) * 34;
            float d = f16le(block);
            int32_t s = 0;
            for (int i = 0; i < 32; i++) s += (int32_t)(int8_t)block[2 + i] * xq[blk * 32 + i];
            inner += d * (float)s;
        }
        acc += dxs[sb] * inner;
    }
    return acc;
}

void orc_q4k_block_ints(const uint8_t *w, const int8_t *qs, const int16_t *bsums, int64_t n, int32_t *isum_out, int32_t *imin_out) {
    for (int64_t b = 0; b < n / 256; b++) {
        const uint8_t *blk = w + b * 144;
        const uint8_t *scales = blk + 4, *q = blk + 16;
        const int8_t *xq = qs + b * 256;
        const int16_t *bs = bsums + b * 8;
        int32_t isum = 0, imin = 0;
        for (int c = 0; c < 4; c++) {
            uint8_t sc1, m1, sc2, m2;
            get_scale_min_k4(2 * c, scales, &sc1, &m1);
            get_scale_min_k4(2 * c + 1, scales, &sc2, &m2);
            int32_t qa = 0, qb = 0;
            for (int l = 0; l < 32; l++) {
                qa += (int32_t)(q[c * 32 + l] & 0xF) * xq[c * 64 + l];
                qb += (int32_t)(q[c * 32 + l] >> 4) * xq[c * 64 + 32 + l];
            }
            isum += (int32_t)sc1 * qa + (int32_t)sc2 * qb;
            imin += (int32_t)m1 * bs[2 * c] + (int32_t)m2 * bs[2 * c + 1];
        }
        isum_out[b] = isum;
        imin_out[b] = imin;
    }
}

void orc_q6k_block_ints(const uint8_t *w, const int8_t *qs, int64_t n, int32_t *isum_out) {
    for (int64_t b = 0; b < n / 256; b++) {
        const uint8_t *blk = w + b * 210;
        const int8_t *xq = qs + b * 256;
        int32_t isum = 0;
        for (int g = 0; g < 2; g++) {
            const uint8_t *ql = blk + g * 64, *qh = blk + 128 + g * 32;
            const int8_t *scs = (const int8_t *)(blk + 192 + g * 8);
            for (int l = 0; l < 32; l++) {
                int32_t q0 = (int32_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
                int32_t q1 = (int32_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int32_t q2 = (int32_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int32_t q3 = (int32_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                int si = l / 16;
                isum += scs[si] * q0 * xq[g * 128 + l] + scs[si + 2] * q1 * xq[g * 128 + 32 + l] +
                        scs[si + 4] * q2 * xq[g * 128 + 64 + l] + scs[si + 6] * q3 * xq[g * 128 + 96 + l];
            }
        }
        isum_out[b] = isum;
    }
}

void orc_q8_0_block_ints(const uint8_t *w, const int8_t *qs, int64_t n, int32_t *s_out) {
    for (int64_t b = 0; b < n / 32; b++) {
        const uint8_t *block = w + b * 34;
        int32_t s = 0;
        for (int i = 0; i < 32; i++) s += (int32_t)(int8_t)block[2 + i] * qs[b * 32 + i];
        s_out[b] = s;
    }
}

/* ------------------------------------------------------------------------ */
/* matvec: Weight::matvec_into (model.rs:218-257) -> matvec_*_into ->
 * parallel_matvec (simd.rs:842-883) -> dot_row (simd.rs:962-1060).  The Q8_K
 * activation is prepared once per call when cols % 256 == 0
 * (prepare_xq_kquant, simd.rs:944-959); Q8_0 falls back to the f32 kernel
 * otherwise, MXFP4 is always scalar f32.  Rows are split in 64-row chunks
 * scheduled dynamically (MATVEC_CHUNK_ROWS, simd.rs:30; MatvecJob
 * simd.rs:1130-1212); a row's value does not depend on the split.            */
static int g_threads = 1;
void orc_set_threads(int threads) { g_threads = threads > 0 ? threads : 1; }
/* 1 (default): the checker's schedule (MXFP4 rows eight at a time, the sink
 * loop's heads on the threads); 0: the reference's own schedule (one row per
 * dot_mxfp4_f32_scalar call in the 64-row worker split, heads one after
 * another), for timing the CPU baseline.  Values are the same either way. */
static int g_fast_schedule = 1;
void orc_set_fast_schedule(int on) { g_fast_schedule = on ? 1 : 0; }

int64_t orc_row_bytes(int dtype, int64_t cols) {
    switch (dtype) {
    case ORC_F32: return cols * 4;
    case ORC_Q8_0: return (cols / 32) * 34;
    case ORC_Q4_K: return (cols / 256) * 144;
    case ORC_Q6_K: return (cols / 256) * 210;
    case ORC_MXFP4: return (cols / 32) * 17;
    default: return 0;
    }
}

/* dot_mxfp4_f32_scalar for 8 rows at once: each row's running sum takes
 * exactly the steps of the one-row function above, in its order
 * (sum += (LUT[n] * scale) * x, element by element); AVX2 lane r is row r.
 * The rows only share the loop, which gives the CPU eight independent add
 * chains instead of one (the checker's speed; no value changes).  Per block
 * each row's 32 values LUT[n] * scale are built in registers (element 2i is
 * the low nibble of byte i, 2i+1 the high one; the table's second half is
 * the first with the sign bit set, -0.0 included, so LUT[n] =
 * LUT[n & 7] | (n & 8) << 28 exactly), then an 8 x 8 transpose per quarter
 * turns them into one vector per element index.  (Shuffles, not gathers:
 * AVX2 gathers are slow on the EPYC hosts of the GPU boxes.) */
__attribute__((target("avx2,fma")))
static inline void transpose8_ps(__m256 *r) {
    __m256 t0 = _mm256_unpacklo_ps(r[0], r[1]), t1 = _mm256_unpackhi_ps(r[0], r[1]);
    __m256 t2 = _mm256_unpacklo_ps(r[2], r[3]), t3 = _mm256_unpackhi_ps(r[2], r[3]);
    __m256 t4 = _mm256_unpacklo_ps(r[4], r[5]), t5 = _mm256_unpackhi_ps(r[4], r[5]);
    __m256 t6 = _mm256_unpacklo_ps(r[6], r[7]), t7 = _mm256_unpackhi_ps(r[6], r[7]);
    __m256 u0 = _mm256_shuffle_ps(t0, t2, 0x44), u1 = _mm256_shuffle_ps(t0, t2, 0xEE);
    __m256 u2 = _mm256_shuffle_ps(t1, t3, 0x44), u3 = _mm256_shuffle_ps(t1, t3, 0xEE);
    __m256 u4 = _mm256_shuffle_ps(t4, t6, 0x44), u5 = _mm256_shuffle_ps(t4, t6, 0xEE);
    __m256 u6 = _mm256_shuffle_ps(t5, t7, 0x44), u7 = _mm256_shuffle_ps(t5, t7, 0xEE);
    r[0] = _mm256_permute2f128_ps(u0, u4, 0x20);
    r[1] = _mm256_permute2f128_ps(u1, u5, 0x20);
    r[2] = _mm256_permute2f128_ps(u2, u6, 0x20);
    r[3] = _mm256_permute2f128_ps(u3, u7, 0x20);
    r[4] = _mm256_permute2f128_ps(u0, u4, 0x31);
    r[5] = _mm256_permute2f128_ps(u1, u5, 0x31);
    r[6] = _mm256_permute2f128_ps(u2, u6, 0x31);
    r[7] = _mm256_permute2f128_ps(u3, u7, 0x31);
}

/* orc_mxfp4_scale for every byte, filled by orc_matvec before its threads
 * start (the same function's values, so nothing changes but the lookup) */
static float g_mxfp4_scale[256];
static int g_mxfp4_scale_ready = 0;
static void mxfp4_scale_table_init(void) {
    if (g_mxfp4_scale_ready) return;
    for (int e = 0; e < 256; e++) g_mxfp4_scale[e] = orc_mxfp4_scale((uint8_t)e);
    g_mxfp4_scale_ready = 1;
}

__attribute__((target("avx2,fma")))
static void dot_mxfp4_f32_scalar_rows8(const uint8_t *w, int64_t rb, const float *x, int64_t n, float *out) {
    const int64_t nb = n / 32;
    const __m256 lut = _mm256_loadu_ps(MXFP4_LUT);
    const __m256i sign = _mm256_set1_epi32((int)0x80000000u);
    const __m128i m4 = _mm_set1_epi8(0x0F);
    __m256 sum = _mm256_setzero_ps();
    for (int64_t b = 0; b < nb; b++) {
        __m256 v[4][8];  /* [quarter][row]: elements 8q..8q+7 of row r */
        for (int r = 0; r < 8; r++) {
            const uint8_t *blk = w + r * rb + b * 17;
            const __m256 sc = _mm256_set1_ps(g_mxfp4_scale[blk[16]]);
            __m128i bytes;
            memcpy(&bytes, blk, 16);
            const __m128i lo = _mm_and_si128(bytes, m4), hi = _mm_and_si128(_mm_srli_epi16(bytes, 4), m4);
            const __m128i e0 = _mm_unpacklo_epi8(lo, hi), e1 = _mm_unpackhi_epi8(lo, hi); /* elements 0..15, 16..31 */
            const __m128i parts[4] = {e0, _mm_srli_si128(e0, 8), e1, _mm_srli_si128(e1, 8)};
            for (int q = 0; q < 4; q++) {
                const __m256i idx = _mm256_cvtepu8_epi32(parts[q]);
                const __m256 val = _mm256_or_ps(_mm256_permutevar8x32_ps(lut, idx),
                                                _mm256_castsi256_ps(_mm256_and_si256(_mm256_slli_epi32(idx, 28), sign)));
                v[q][r] = _mm256_mul_ps(val, sc);
            }
        }
        const float *xb = x + b * 32;
        for (int q = 0; q < 4; q++) {
            transpose8_ps(v[q]);
            for (int jj = 0; jj < 8; jj++)
                sum = _mm256_add_ps(sum, _mm256_mul_ps(v[q][jj], _mm256_set1_ps(xb[q * 8 + jj])));
        }
    }
    _mm256_storeu_ps(out, sum);
}

void orc_matvec(int dtype, const uint8_t *w, const float *x, int64_t rows, int64_t cols, float *out, int threads) {
    if (threads <= 0) threads = g_threads;
    int64_t rb = orc_row_bytes(dtype, cols);
    if (dtype == ORC_MXFP4 && g_fast_schedule) {
        /* scheduling only: groups of 8 rows, each row's value as the
         * one-row kernel's (a row's value does not depend on the split) */
        mxfp4_scale_table_init();
        if (threads > rows) threads = (int)rows;
        int serial = threads <= 1 || rows < (int64_t)threads * 8;
        int64_t groups = rows / 8;
#pragma omp parallel for schedule(dynamic, 8) num_threads(threads) if (!serial)
        for (int64_t gi = 0; gi < groups; gi++) dot_mxfp4_f32_scalar_rows8(w + gi * 8 * rb, rb, x, cols, out + gi * 8);
        for (int64_t r = groups * 8; r < rows; r++) out[r] = orc_dot_mxfp4_f32_scalar(w + r * rb, x, cols);
        return;
    }
    int use_xq = (dtype == ORC_Q8_0 || dtype == ORC_Q4_K || dtype == ORC_Q6_K) && cols >= 256 && cols % 256 == 0;
    int8_t *qs = NULL;
    float *dx = NULL;
    int16_t *bs = NULL;
    if (use_xq) {
        qs = (int8_t *)malloc((size_t)cols);
        dx = (float *)malloc((size_t)(cols / 256) * 4);
        bs = (int16_t *)malloc((size_t)(cols / 32) * 2);
        orc_quantize_row_q8k_avx2(x, cols, qs, dx, bs);
    }
    if (threads > rows) threads = (int)rows;
    int serial = threads <= 1 || rows < (int64_t)threads * 8;
#pragma omp parallel for schedule(dynamic, 64) num_threads(threads) if (!serial)
    for (int64_t r = 0; r < rows; r++) {
        const uint8_t *row = w + r * rb;
        float v;
        switch (dtype) {
        case ORC_F32: v = orc_dot_f32_avx2((const float *)row, x, cols); break;
        case ORC_Q8_0: v = use_xq ? orc_dot_q8_0_q8k_avx2(row, qs, dx, bs, cols) : orc_dot_q8_0_f32_avx2(row, x, cols); break;
        case ORC_Q4_K: v = orc_dot_q4_k_q8k_avx2(row, qs, dx, bs, cols); break;
        case ORC_Q6_K: v = orc_dot_q6_k_q8k_avx2(row, qs, dx, bs, cols); break;
        case ORC_MXFP4: v = orc_dot_mxfp4_f32_scalar(row, x, cols); break;
        default: v = 0.0f;
        }
        out[r] = v;
    }
    free(qs);
    free(dx);
    free(bs);
}

/* ------------------------------------------------------------------------ */
/* attention, model.rs:5739-6198.  exp_attn (model.rs:5720-5726) is f32::exp,
 * i.e. libm expf.                                                            */
static inline int linear_slots(int64_t s, int64_t e, int64_t slots) { return s <= e && e < slots; }

int64_t orc_attention_start_pos(int64_t pos, int64_t window) {
    /* model.rs:1511-1520 */
    if (window > 0) {
        int64_t v = pos + 1 - window;
        return v > 0 ? v : 0;
    }
    return 0;
}

static void online_attention_impl(const float *q, const float *keys, const float *values,
                                  int64_t ks, int64_t vs, int64_t slots, int64_t hd, int64_t vd,
                                  int64_t start_t, int64_t end_t, float scale, int use_sink,
                                  float sink, float *out) {
    if (slots == 0 || start_t > end_t) return;
    float max_score = use_sink ? sink : -INFINITY;
    float denom = use_sink ? 1.0f : 0.0f;
    int64_t slot = linear_slots(start_t, end_t, slots) ? start_t : start_t % slots;
    for (int64_t t = start_t; t <= end_t; t++) {
        const float *krow = keys + slot * ks;
        float score = orc_dot_f32_avx2(q, krow, hd) * scale;
        const float *vrow = values + slot * vs;
        if (score > max_score) {
            float old_scale = isfinite(max_score) ? expf(max_score - score) : 0.0f;
            scale_add_f32_avx2(out, old_scale, vrow, vd);
            denom = denom * old_scale + 1.0f;
            max_score = score;
        } else {
            float weight = expf(score - max_score);
            axpy_f32_avx2(out, weight, vrow, vd);
            denom += weight;
        }
        slot++;
        if (slot == slots) slot = 0;
    }
    if (denom > 0.0f) scale_f32_avx2(out, 1.0f / denom, vd);
}

/* online_attention, model.rs:5807-5869 */
void orc_online_attention(const float *q, const float *keys, const float *values, int64_t ks, int64_t vs,
                          int64_t slots, int64_t hd, int64_t vd, int64_t start_t, int64_t end_t,
                          float scale, float *out) {
    online_attention_impl(q, keys, values, ks, vs, slots, hd, vd, start_t, end_t, scale, 0, 0.0f, out);
}

/* online_attention_with_sink, model.rs:5739-5803 */
void orc_online_attention_with_sink(const float *q, const float *keys, const float *values, int64_t ks,
                                    int64_t vs, int64_t slots, int64_t hd, int64_t vd, int64_t start_t,
                                    int64_t end_t, float scale, float sink, float *out) {
    online_attention_impl(q, keys, values, ks, vs, slots, hd, vd, start_t, end_t, scale, 1, sink, out);
}

#define MAX_KV_MUL 16
/* online_attention_grouped, model.rs:6034-6191 */
void orc_online_attention_grouped(const float *queries, const float *keys, const float *values, int64_t ks,
                                  int64_t vs, int64_t slots, int64_t hd, int64_t vd, int64_t kv_mul,
                                  int64_t start_t, int64_t end_t, float scale, float *out) {
    if (slots == 0 || start_t > end_t) return;
    if (kv_mul == 1) {
        orc_online_attention(queries, keys, values, ks, vs, slots, hd, vd, start_t, end_t, scale, out);
        return;
    }
    float max_score[MAX_KV_MUL], denom[MAX_KV_MUL];
    for (int g = 0; g < MAX_KV_MUL; g++) {
        max_score[g] = -INFINITY;
        denom[g] = 0.0f;
    }
    if (kv_mul > MAX_KV_MUL) kv_mul = MAX_KV_MUL;
    int64_t slot = linear_slots(start_t, end_t, slots) ? start_t : start_t % slots;
    for (int64_t t = start_t; t <= end_t; t++) {
        const float *krow = keys + slot * ks;
        const float *vrow = values + slot * vs;
        if (kv_mul == 4 || kv_mul == 6) {
            float scores[4];
            dot_f32x4_avx2(queries, queries + hd, queries + 2 * hd, queries + 3 * hd, krow, hd, scores);
            float multiplier[4] = {1.0f, 1.0f, 1.0f, 1.0f};
            float alpha[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int g = 0; g < 4; g++) {
                float score = scores[g] * scale;
                if (score > max_score[g]) {
                    float old_scale = isfinite(max_score[g]) ? expf(max_score[g] - score) : 0.0f;
                    multiplier[g] = old_scale;
                    alpha[g] = 1.0f;
                    denom[g] = denom[g] * old_scale + 1.0f;
                    max_score[g] = score;
                } else {
                    alpha[g] = expf(score - max_score[g]);
                    denom[g] += alpha[g];
                }
            }
            affine_add_f32x4_avx2(out, out + vd, out + 2 * vd, out + 3 * vd, multiplier, alpha, vrow, vd);
            if (kv_mul == 6) {
                for (int g = 4; g < 6; g++) {
                    float score = orc_dot_f32_avx2(queries + g * hd, krow, hd) * scale;
                    float *o = out + g * vd;
                    if (score > max_score[g]) {
                        float old_scale = isfinite(max_score[g]) ? expf(max_score[g] - score) : 0.0f;
                        scale_add_f32_avx2(o, old_scale, vrow, vd);
                        denom[g] = denom[g] * old_scale + 1.0f;
                        max_score[g] = score;
                    } else {
                        float weight = expf(score - max_score[g]);
                        axpy_f32_avx2(o, weight, vrow, vd);
                        denom[g] += weight;
                    }
                }
            }
        } else {
            for (int64_t g = 0; g < kv_mul; g++) {
                float score = orc_dot_f32_avx2(queries + g * hd, krow, hd) * scale;
                float *o = out + g * vd;
                if (score > max_score[g]) {
                    float old_scale = isfinite(max_score[g]) ? expf(max_score[g] - score) : 0.0f;
                    scale_add_f32_avx2(o, old_scale, vrow, vd);
                    denom[g] = denom[g] * old_scale + 1.0f;
                    max_score[g] = score;
                } else {
                    float weight = expf(score - max_score[g]);
                    axpy_f32_avx2(o, weight, vrow, vd);
                    denom[g] += weight;
                }
            }
        }
        slot++;
        if (slot == slots) slot = 0;
    }
    for (int64_t g = 0; g < kv_mul; g++)
        if (denom[g] > 0.0f) scale_f32_avx2(out + g * vd, 1.0f / denom[g], vd);
}

/* attention_over_kv_heads, model.rs:5952-6026 (serial and parallel paths are
 * equivalent: each KV head writes a disjoint band).                          */
void orc_attention_over_kv_heads(const float *q, const float *keys, const float *values, int64_t ks,
                                 int64_t vs, int64_t slots, int64_t hd, int64_t vd, int64_t n_kv,
                                 int64_t kv_mul, int64_t start_t, int64_t end_t, float scale, float *out) {
    int nt = g_threads < (int)n_kv ? g_threads : (int)n_kv;
    int64_t work = (end_t >= start_t ? end_t - start_t + 1 : 0) * n_kv;
#pragma omp parallel for schedule(static) num_threads(nt > 0 ? nt : 1) if (n_kv > 1 && nt > 1 && work >= 4096)
    for (int64_t h = 0; h < n_kv; h++) {
        orc_online_attention_grouped(q + h * kv_mul * hd, keys + h * hd, values + h * vd, ks, vs, slots, hd, vd,
                                     kv_mul, start_t, end_t, scale, out + h * kv_mul * vd);
    }
}

/* ------------------------------------------------------------------------ */
/* bf16 KV cache (KVCache::enable_bf16, model.rs:1406-1421; attention,
 * model.rs:6205-6580).  bf16_to_f32 is exact (simd.rs:82-85), so the
 * reference's widened-row kernels axpy_bf16_f32, scale_add_bf16_f32 and
 * affine_add_bf16x4_f32 (simd.rs:7314-7440) are the f32 kernels above on the
 * widened row, element for element; dot_bf16x4_f32 is dot_f32x4 on the
 * widened key.  dot_bf16_f32 (simd.rs:7292-7311) has an order of its own:
 * one 8-wide accumulator, hsum_avx, then the scalar tail. */
uint16_t orc_f32_to_bf16(float x) {
    /* simd.rs:88-96: round to nearest even; NaN keeps its payload, quiet */
    uint32_t bits;
    memcpy(&bits, &x, 4);
    if (isnan(x)) return (uint16_t)((bits >> 16) | 0x0040);
    uint32_t rounded = bits + 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(rounded >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

static void bf16_widen(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = orc_bf16_to_f32(src[i]);
}

/* dot_bf16_f32_avx2, simd.rs:7292-7311 (on the widened key row) */
__attribute__((target("avx2,fma")))
float orc_dot_bf16_f32_avx2(const float *a, const float *bw, int64_t n) {
    int64_t main_ = n / 8;
    __m256 acc = _mm256_setzero_ps();
    for (int64_t i = 0; i < main_; i++)
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + 8 * i), _mm256_loadu_ps(bw + 8 * i), acc);
    float sum = hsum_avx(acc);
    for (int64_t i = main_ * 8; i < n; i++) sum += a[i] * bw[i];
    return sum;
}

#define BF16_MAX_DIM 512
/* online_attention_bf16, model.rs:6219-6276 */
static void online_attention_bf16(const float *q, const uint16_t *keys, const uint16_t *values, int64_t ks,
                                  int64_t vs, int64_t slots, int64_t hd, int64_t vd, int64_t start_t, int64_t end_t,
                                  float scale, float *out) {
    if (slots == 0 || start_t > end_t) return;
    float kw[BF16_MAX_DIM], vw[BF16_MAX_DIM];
    float max_score = -INFINITY, denom = 0.0f;
    int64_t slot = linear_slots(start_t, end_t, slots) ? start_t : start_t % slots;
    for (int64_t t = start_t; t <= end_t; t++) {
        bf16_widen(keys + slot * ks, kw, hd);
        bf16_widen(values + slot * vs, vw, vd);
        float score = orc_dot_bf16_f32_avx2(q, kw, hd) * scale;
        if (score > max_score) {
            float old_scale = isfinite(max_score) ? expf(max_score - score) : 0.0f;
            scale_add_f32_avx2(out, old_scale, vw, vd);
            denom = denom * old_scale + 1.0f;
            max_score = score;
        } else {
            float weight = expf(score - max_score);
            axpy_f32_avx2(out, weight, vw, vd);
            denom += weight;
        }
        slot++;
        if (slot == slots) slot = 0;
    }
    if (denom > 0.0f) scale_f32_avx2(out, 1.0f / denom, vd);
}

/* online_attention_grouped_bf16, model.rs:6278-6437 */
void orc_online_attention_grouped_bf16(const float *queries, const uint16_t *keys, const uint16_t *values, int64_t ks,
                                       int64_t vs, int64_t slots, int64_t hd, int64_t vd, int64_t kv_mul,
                                       int64_t start_t, int64_t end_t, float scale, float *out) {
    if (slots == 0 || start_t > end_t) return;
    if (kv_mul == 1) {
        online_attention_bf16(queries, keys, values, ks, vs, slots, hd, vd, start_t, end_t, scale, out);
        return;
    }
    if (kv_mul > MAX_KV_MUL) kv_mul = MAX_KV_MUL;
    float kw[BF16_MAX_DIM], vw[BF16_MAX_DIM];
    float max_score[MAX_KV_MUL], denom[MAX_KV_MUL];
    for (int g = 0; g < MAX_KV_MUL; g++) {
        max_score[g] = -INFINITY;
        denom[g] = 0.0f;
    }
    int64_t slot = linear_slots(start_t, end_t, slots) ? start_t : start_t % slots;
    for (int64_t t = start_t; t <= end_t; t++) {
        bf16_widen(keys + slot * ks, kw, hd);
        bf16_widen(values + slot * vs, vw, vd);
        if (kv_mul == 4 || kv_mul == 6) {
            float scores[4];
            dot_f32x4_avx2(queries, queries + hd, queries + 2 * hd, queries + 3 * hd, kw, hd, scores);
            float multiplier[4] = {1.0f, 1.0f, 1.0f, 1.0f}, alpha[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int g = 0; g < 4; g++) {
                float score = scores[g] * scale;
                if (score > max_score[g]) {
                    float old_scale = isfinite(max_score[g]) ? expf(max_score[g] - score) : 0.0f;
                    multiplier[g] = old_scale;
                    alpha[g] = 1.0f;
                    denom[g] = denom[g] * old_scale + 1.0f;
                    max_score[g] = score;
                } else {
                    alpha[g] = expf(score - max_score[g]);
                    denom[g] += alpha[g];
                }
            }
            affine_add_f32x4_avx2(out, out + vd, out + 2 * vd, out + 3 * vd, multiplier, alpha, vw, vd);
            for (int64_t g = 4; g < kv_mul; g++) {
                float score = orc_dot_bf16_f32_avx2(queries + g * hd, kw, hd) * scale;
                float *o = out + g * vd;
                if (score > max_score[g]) {
                    float old_scale = isfinite(max_score[g]) ? expf(max_score[g] - score) : 0.0f;
                    scale_add_f32_avx2(o, old_scale, vw, vd);
                    denom[g] = denom[g] * old_scale + 1.0f;
                    max_score[g] = score;
                } else {
                    float weight = expf(score - max_score[g]);
                    axpy_f32_avx2(o, weight, vw, vd);
                    denom[g] += weight;
                }
            }
        } else {
            for (int64_t g = 0; g < kv_mul; g++) {
                float score = orc_dot_bf16_f32_avx2(queries + g * hd, kw, hd) * scale;
                float *o = out + g * vd;
                if (score > max_score[g]) {
                    float old_scale = isfinite(max_score[g]) ? expf(max_score[g] - score) : 0.0f;
                    scale_add_f32_avx2(o, old_scale, vw, vd);
                    denom[g] = denom[g] * old_scale + 1.0f;
                    max_score[g] = score;
                } else {
                    float weight = expf(score - max_score[g]);
                    axpy_f32_avx2(o, weight, vw, vd);
                    denom[g] += weight;
                }
            }
        }
        slot++;
        if (slot == slots) slot = 0;
    }
    for (int64_t g = 0; g < kv_mul; g++)
        if (denom[g] > 0.0f) scale_f32_avx2(out + g * vd, 1.0f / denom[g], vd);
}

/* attention_over_kv_heads_bf16, model.rs:6508-6580 */
void orc_attention_over_kv_heads_bf16(const float *q, const uint16_t *keys, const uint16_t *values, int64_t ks,
                                      int64_t vs, int64_t slots, int64_t hd, int64_t vd, int64_t n_kv,
                                      int64_t kv_mul, int64_t start_t, int64_t end_t, float scale, float *out) {
    int nt = g_threads < (int)n_kv ? g_threads : (int)n_kv;
    int64_t work = (end_t >= start_t ? end_t - start_t + 1 : 0) * n_kv;
#pragma omp parallel for schedule(static) num_threads(nt > 0 ? nt : 1) if (n_kv > 1 && nt > 1 && work >= 4096)
    for (int64_t h = 0; h < n_kv; h++) {
        orc_online_attention_grouped_bf16(q + h * kv_mul * hd, keys + h * hd, values + h * vd, ks, vs, slots, hd, vd,
                                          kv_mul, start_t, end_t, scale, out + h * kv_mul * vd);
    }
}

/* per-head sink attention loop, model.rs:6812-6833 (output zeroed first) */
/* The gpt-oss per-head sink loop (model.rs:6812-6833).  The reference runs
 * the heads one after another; each writes only its own output band, so the
 * checker runs them on its threads with the same values. */
void orc_attention_sink_heads(const float *q, const float *keys, const float *values, const float *sinks,
                              int64_t ks, int64_t vs, int64_t slots, int64_t hd, int64_t vd, int64_t n_heads,
                              int64_t kv_mul, int64_t start_t, int64_t end_t, float scale, float *out) {
    memset(out, 0, (size_t)(n_heads * vd) * 4);
    int nt = g_threads < (int)n_heads ? g_threads : (int)n_heads;
    int64_t work = (end_t >= start_t ? end_t - start_t + 1 : 0) * n_heads;
#pragma omp parallel for schedule(static) num_threads(nt > 0 ? nt : 1) \
    if (g_fast_schedule && n_heads > 1 && nt > 1 && work >= 4096)
    for (int64_t h = 0; h < n_heads; h++) {
        int64_t kvh = h / kv_mul;
        orc_online_attention_with_sink(q + h * hd, keys + kvh * hd, values + kvh * vd, ks, vs, slots, hd, vd,
                                       start_t, end_t, scale, sinks[h], out + h * vd);
    }
}

/* ------------------------------------------------------------------------ */
/* rms_norm_into, model.rs:5429-5437 */
void orc_rms_norm(const float *x, const float *w, float eps, int64_t n, float *out) {
    float ss = orc_dot_f32_avx2(x, x, n) / (float)n;
    float scale = 1.0f / sqrtf(ss + eps);
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* build_rope_inv_freq_with_factors, model.rs:3035-3057 (no factors) */
void orc_build_rope_inv_freq(float theta, int64_t head_dim, float scaling, float *inv) {
    for (int64_t pair = 0; pair < head_dim / 2; pair++) {
        float i = (float)(pair * 2);
        float base_freq = powf(theta, i / (float)head_dim);
        inv[pair] = 1.0f / (scaling * base_freq * 1.0f);
    }
}

/* build_rope_inv_freq_gpt_oss, model.rs:3059-3098: YaRN inverse frequencies
 * (a linear ramp between the extrapolated 1/base and the interpolated
 * 1/(scaling*base) over pairs low..high) and the concentration
 * 0.1*ln(scaling) + 1, in f32 with libm logf/powf as Rust's f32::ln/powf. */
void orc_build_rope_inv_freq_gpt_oss(float theta, int64_t head_dim, float scaling, int64_t orig_ctx, float *inv,
                                     float *concentration) {
    const float pi = 3.14159265358979323846f;
    float d_half = (float)head_dim / 2.0f;
    float low = 0.0f, high = 0.0f;
    if (scaling > 1.0f) {
        low = d_half * (logf((float)orig_ctx / (32.0f * 2.0f * pi)) / logf(theta));
        high = d_half * (logf((float)orig_ctx / (1.0f * 2.0f * pi)) / logf(theta));
    }
    *concentration = scaling > 1.0f ? 0.1f * logf(scaling) + 1.0f : 1.0f;
    for (int64_t pair = 0; pair < head_dim / 2; pair++) {
        float i = (float)(pair * 2);
        float base_freq = powf(theta, i / (float)head_dim);
        if (scaling > 1.0f) {
            float idx = (float)pair;
            float ramp = (idx - low) / (high - low);
            ramp = ramp < 0.0f ? 0.0f : (ramp > 1.0f ? 1.0f : ramp);
            float mask = 1.0f - ramp;
            float interpolation = 1.0f / (scaling * base_freq);
            float extrapolation = 1.0f / base_freq;
            inv[pair] = interpolation * (1.0f - mask) + extrapolation * mask;
        } else {
            inv[pair] = 1.0f / base_freq;
        }
    }
}

/* apply_rope_qk, model.rs:5562-5603 (adjacent pairs) */
void orc_rope_qk(float *q, float *k, int64_t pos, int64_t hd, int64_t nh, int64_t nkv, const float *inv_freq) {
    int64_t last = hd - (hd % 2);
    for (int64_t i = 0; i < last; i += 2) {
        float angle = (float)pos * inv_freq[i / 2];
        float s = sinf(angle), c = cosf(angle);
        for (int64_t h = 0; h < nh; h++) {
            float *p = q + h * hd + i;
            float v0 = p[0], v1 = p[1];
            p[0] = v0 * c - v1 * s;
            p[1] = v0 * s + v1 * c;
        }
        for (int64_t h = 0; h < nkv; h++) {
            float *p = k + h * hd + i;
            float v0 = p[0], v1 = p[1];
            p[0] = v0 * c - v1 * s;
            p[1] = v0 * s + v1 * c;
        }
    }
}

/* apply_rope_gpt_oss, model.rs:6603-6636: adjacent pairs, with cos and sin
 * scaled by the YaRN concentration before the rotation. */
void orc_rope_gpt_oss(float *q, float *k, int64_t pos, int64_t hd, int64_t nh, int64_t nkv, float concentration,
                      const float *inv_freq) {
    for (int64_t i = 0; i < hd; i += 2) {
        float angle = (float)pos * inv_freq[i / 2];
        float s = sinf(angle) * concentration, c = cosf(angle) * concentration;
        for (int64_t h = 0; h < nh; h++) {
            float *p = q + h * hd + i;
            float v0 = p[0], v1 = p[1];
            p[0] = v0 * c - v1 * s;
            p[1] = v0 * s + v1 * c;
        }
        for (int64_t h = 0; h < nkv; h++) {
            float *p = k + h * hd + i;
            float v0 = p[0], v1 = p[1];
            p[0] = v0 * c - v1 * s;
            p[1] = v0 * s + v1 * c;
        }
    }
}

/* apply_rope_qk_neox, model.rs:5606-5647 (rotate-half pairs) */
void orc_rope_qk_neox(float *q, float *k, int64_t pos, int64_t hd, int64_t nh, int64_t nkv, const float *inv_freq) {
    int64_t half = hd / 2;
    for (int64_t i = 0; i < half; i++) {
        float angle = (float)pos * inv_freq[i];
        float s = sinf(angle), c = cosf(angle);
        for (int64_t h = 0; h < nh; h++) {
            float *p = q + h * hd;
            float v0 = p[i], v1 = p[i + half];
            p[i] = v0 * c - v1 * s;
            p[i + half] = v0 * s + v1 * c;
        }
        for (int64_t h = 0; h < nkv; h++) {
            float *p = k + h * hd;
            float v0 = p[i], v1 = p[i + half];
            p[i] = v0 * c - v1 * s;
            p[i + half] = v0 * s + v1 * c;
        }
    }
}

/* silu_mul: scalar simd.rs:2393-2399; AVX2 simd.rs:2468-2484 with the
 * Cephes-style expf of simd.rs:2406-2464 (constants from simd.rs:2410-2421). */
void orc_silu_mul_scalar(const float *gate, const float *up, float *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float g = gate[i];
        out[i] = g / (1.0f + expf(-g)) * up[i];
    }
}

__attribute__((target("avx2,fma")))
static inline __m256 exp_ps_avx2(__m256 x) {
    x = _mm256_min_ps(_mm256_set1_ps(88.37626f), _mm256_max_ps(_mm256_set1_ps(-88.37626f), x));
    __m256 fx = _mm256_fmadd_ps(x, _mm256_set1_ps(1.44269504088896340736f), _mm256_set1_ps(0.5f));
    fx = _mm256_floor_ps(fx);
    x = _mm256_fnmadd_ps(fx, _mm256_set1_ps(0.6933594f), x);
    x = _mm256_fnmadd_ps(fx, _mm256_set1_ps(-2.1219444e-4f), x);
    __m256 y = _mm256_set1_ps(1.9875691e-4f);
    y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(1.3982e-3f));
    y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(8.333452e-3f));
    y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(4.1665796e-2f));
    y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(1.6666665e-1f));
    y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(0.5f));
    __m256 x2 = _mm256_mul_ps(x, x);
    y = _mm256_add_ps(_mm256_fmadd_ps(y, x2, x), _mm256_set1_ps(1.0f));
    __m256i nn = _mm256_cvttps_epi32(fx);
    __m256 pow2n = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_add_epi32(nn, _mm256_set1_epi32(0x7f)), 23));
    return _mm256_mul_ps(y, pow2n);
}

__attribute__((target("avx2,fma")))
void orc_silu_mul_avx2(const float *gate, const float *up, float *out, int64_t n) {
    int64_t main_ = n / 8 * 8;
    __m256 one = _mm256_set1_ps(1.0f);
    for (int64_t i = 0; i < main_; i += 8) {
        __m256 g = _mm256_loadu_ps(gate + i);
        __m256 u = _mm256_loadu_ps(up + i);
        __m256 e = exp_ps_avx2(_mm256_sub_ps(_mm256_setzero_ps(), g));
        __m256 s = _mm256_div_ps(g, _mm256_add_ps(one, e));
        _mm256_storeu_ps(out + i, _mm256_mul_ps(s, u));
    }
    orc_silu_mul_scalar(gate + main_, up + main_, out + main_, n - main_);
}

/* swiglu_gpt_oss, model.rs:6596-6600 */
float orc_swiglu_gpt_oss(float g, float u) {
    g = fminf(g, 7.0f);
    u = u < -7.0f ? -7.0f : (u > 7.0f ? 7.0f : u);
    return g * (1.0f / (1.0f + expf(-1.702f * g))) * (u + 1.0f);
}

/* total_cmp order of f32 (used by the router, model.rs:6672, 6712) */
static inline int32_t total_key(float v) {
    int32_t b;
    memcpy(&b, &v, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

/* select_top_logits_into + bubble_up_router_last, model.rs:6659-6716 */
void orc_select_top_logits(const float *logits, int64_t n, int64_t k, int32_t *idx, float *val) {
    int64_t len = 0;
    if (k == 0) return;
    for (int64_t i = 0; i < n; i++) {
        float v = logits[i];
        if (len < k) {
            idx[len] = (int32_t)i;
            val[len] = v;
            len++;
        } else if (total_key(v) > total_key(val[len - 1])) {
            idx[len - 1] = (int32_t)i;
            val[len - 1] = v;
        } else {
            continue;
        }
        int64_t j = len - 1;
        while (j > 0 && total_key(val[j]) > total_key(val[j - 1])) {
            int32_t ti = idx[j];
            idx[j] = idx[j - 1];
            idx[j - 1] = ti;
            float tv = val[j];
            val[j] = val[j - 1];
            val[j - 1] = tv;
            j--;
        }
    }
}

/* softmax_selected_into, model.rs:6639-6656 */
void orc_softmax_selected(const float *val, int64_t k, float *out) {
    float mx = -INFINITY;
    for (int64_t i = 0; i < k; i++) mx = fmaxf(mx, val[i]);
    float sum = 0.0f;
    for (int64_t i = 0; i < k; i++) {
        out[i] = expf(val[i] - mx);
        sum += out[i];
    }
    if (sum > 0.0f)
        for (int64_t i = 0; i < k; i++) out[i] /= sum;
}

/* apply_repeat_penalty / argmax_finite_token, sampling.rs:321-356 */
void orc_apply_repeat_penalty(float *logits, int64_t n, const uint32_t *recent, int64_t nrecent, float penalty) {
    if (penalty == 1.0f) return;
    for (int64_t i = 0; i < nrecent; i++) {
        uint32_t tok = recent[i];
        if ((int64_t)tok < n) {
            float v = logits[tok];
            logits[tok] = !isfinite(v) ? -INFINITY : (v > 0.0f ? v / penalty : v * penalty);
        }
    }
}

uint32_t orc_argmax_finite(const float *logits, int64_t n) {
    if (n == 0) return 0;
    int64_t best = 0;
    float bv = isfinite(logits[0]) ? logits[0] : -INFINITY;
    for (int64_t i = 1; i < n; i++) {
        float v = isfinite(logits[i]) ? logits[i] : -INFINITY;
        if (v > bv) {
            bv = v;
            best = i;
        }
    }
    return (uint32_t)best;
}

/* greedy branch of sample_with_scratch, sampling.rs:78-83 */
uint32_t orc_greedy(float *logits, int64_t n, const uint32_t *recent, int64_t nrecent, float penalty) {
    if (n == 0) return 0;
    orc_apply_repeat_penalty(logits, n, recent, nrecent, penalty);
    return orc_argmax_finite(logits, n);
}

/* ------------------------------------------------------------------------ */
/* Standard decode model: forward_into, model.rs:7177-7358, with KVCache
 * (model.rs:1328-1525) and the decode loop's recent-token window
 * (runtime.rs:493-521, RECENT_TOKEN_LIMIT = 64).                             */
struct orc_model {
    orc_config c;
    orc_layer *layers;
    const float *output_norm;
    const uint8_t *output_w;
    uint32_t output_type;
    const uint8_t *embd;
    uint32_t embd_type;
    float *inv_freq;
    float **k, **v;
    float *x, *xn, *q, *kk, *vv, *attn, *proj, *gate, *up, *hidden;
};

orc_model *orc_model_create(const orc_config *cfg) {
    orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
    m->c = *cfg;
    int64_t kdim = (int64_t)cfg->n_kv_heads * cfg->head_dim;
    int64_t vdim = (int64_t)cfg->n_kv_heads * cfg->value_dim;
    m->layers = (orc_layer *)calloc((size_t)cfg->n_layers, sizeof(orc_layer));
    m->k = (float **)calloc((size_t)cfg->n_layers, sizeof(float *));
    m->v = (float **)calloc((size_t)cfg->n_layers, sizeof(float *));
    /* bf16 storage holds uint16 elements in the same buffers (enable_bf16) */
    const size_t esz = cfg->kv_bf16 ? 2 : 4;
    for (int l = 0; l < cfg->n_layers; l++) {
        m->k[l] = (float *)calloc((size_t)(cfg->storage_len * kdim), esz);
        m->v[l] = (float *)calloc((size_t)(cfg->storage_len * vdim), esz);
    }
    int64_t dim = cfg->dim;
    m->x = (float *)calloc((size_t)dim, 4);
    m->xn = (float *)calloc((size_t)dim, 4);
    m->q = (float *)calloc((size_t)cfg->n_heads * cfg->head_dim, 4);
    m->kk = (float *)calloc((size_t)kdim, 4);
    m->vv = (float *)calloc((size_t)vdim, 4);
    m->attn = (float *)calloc((size_t)cfg->n_heads * cfg->value_dim, 4);
    m->proj = (float *)calloc((size_t)(dim > cfg->hidden_dim ? dim : cfg->hidden_dim), 4);
    m->gate = (float *)calloc((size_t)cfg->hidden_dim, 4);
    m->up = (float *)calloc((size_t)cfg->hidden_dim, 4);
    m->hidden = (float *)calloc((size_t)cfg->hidden_dim, 4);
    m->inv_freq = (float *)calloc((size_t)cfg->head_dim, 4);
    return m;
}

void orc_model_free(orc_model *m) {
    if (!m) return;
    for (int l = 0; l < m->c.n_layers; l++) {
        free(m->k[l]);
        free(m->v[l]);
    }
    free(m->k); free(m->v); free(m->layers);
    free(m->x); free(m->xn); free(m->q); free(m->kk); free(m->vv); free(m->attn);
    free(m->proj); free(m->gate); free(m->up); free(m->hidden); free(m->inv_freq);
    free(m);
}

int orc_model_set_layer(orc_model *m, int32_t l, const orc_layer *layer) {
    if (l < 0 || l >= m->c.n_layers) return 0;
    m->layers[l] = *layer;
    return 1;
}

int orc_model_set_output(orc_model *m, const float *output_norm, const uint8_t *output_w, uint32_t output_type,
                         const uint8_t *embd, uint32_t embd_type, const float *inv_freq) {
    m->output_norm = output_norm;
    m->output_w = output_w;
    m->output_type = output_type;
    m->embd = embd;
    m->embd_type = embd_type;
    memcpy(m->inv_freq, inv_freq, (size_t)(m->c.head_dim / 2) * 4);
    return 1;
}

float *orc_model_kv(orc_model *m, int32_t layer, int32_t which) { return which ? m->v[layer] : m->k[layer]; }

static void add_bias(float *out, const float *b, uint32_t len) {
    if (!b || !len) return;
    for (uint32_t i = 0; i < len; i++) out[i] += b[i];
}

/* forward_into (model.rs:7177-7358).  start_t >= 0 fixes every layer's
 * attention start as the Metal resident decoder's start_t argument does
 * (metal_backend.m:2167-2189); start_t < 0 takes attention_start_pos. */
void orc_model_forward_from(orc_model *m, uint32_t token, int64_t pos, int64_t start_t, float *logits,
                            int want_logits) {
    const orc_config *c = &m->c;
    int64_t dim = c->dim, hd = c->head_dim, vd = c->value_dim;
    int64_t kdim = (int64_t)c->n_kv_heads * hd, vdim = (int64_t)c->n_kv_heads * vd;
    int64_t kv_mul = c->n_heads / c->n_kv_heads;
    int th = g_threads;
    /* token_embd.row_into (model.rs:7193, 267-289) */
    orc_dequant_row((int)m->embd_type, m->embd + (int64_t)token * orc_row_bytes((int)m->embd_type, dim), m->x, dim);
    int64_t window = c->sliding_window;
    int64_t slot = window > 0 ? pos % c->storage_len : pos; /* slot_for_pos, model.rs:1458-1464 */
    for (int l = 0; l < c->n_layers; l++) {
        const orc_layer *L = &m->layers[l];
        orc_rms_norm(m->x, L->attn_norm, c->eps, dim, m->xn);
        orc_matvec((int)L->w_type[0], L->w[0], m->xn, L->w_rows[0], dim, m->q, th);
        orc_matvec((int)L->w_type[1], L->w[1], m->xn, L->w_rows[1], dim, m->kk, th);
        orc_matvec((int)L->w_type[2], L->w[2], m->xn, L->w_rows[2], dim, m->vv, th);
        add_bias(m->q, L->bq, L->bq_len);
        add_bias(m->kk, L->bk, L->bk_len);
        add_bias(m->vv, L->bv, L->bv_len);
        if (c->neox)
            orc_rope_qk_neox(m->q, m->kk, pos, hd, c->n_heads, c->n_kv_heads, m->inv_freq);
        else
            orc_rope_qk(m->q, m->kk, pos, hd, c->n_heads, c->n_kv_heads, m->inv_freq);
        float scale = 1.0f / sqrtf((float)hd);
        int64_t start = start_t >= 0 ? start_t : orc_attention_start_pos(pos, window);
        if (c->kv_bf16) {
            /* KVCache::write_k / write_v narrow to bf16 (model.rs:1478-1502);
             * forward_into then takes attention_over_kv_heads_bf16 (:7245-7261) */
            uint16_t *kc = (uint16_t *)m->k[l] + slot * kdim, *vc = (uint16_t *)m->v[l] + slot * vdim;
            for (int64_t i = 0; i < kdim; i++) kc[i] = orc_f32_to_bf16(m->kk[i]);
            for (int64_t i = 0; i < vdim; i++) vc[i] = orc_f32_to_bf16(m->vv[i]);
            orc_attention_over_kv_heads_bf16(m->q, (const uint16_t *)m->k[l], (const uint16_t *)m->v[l], kdim, vdim,
                                             c->storage_len, hd, vd, c->n_kv_heads, kv_mul, start, pos, scale, m->attn);
        } else {
            memcpy(m->k[l] + slot * kdim, m->kk, (size_t)kdim * 4);
            memcpy(m->v[l] + slot * vdim, m->vv, (size_t)vdim * 4);
            orc_attention_over_kv_heads(m->q, m->k[l], m->v[l], kdim, vdim, c->storage_len, hd, vd, c->n_kv_heads,
                                        kv_mul, start, pos, scale, m->attn);
        }
        orc_matvec((int)L->w_type[3], L->w[3], m->attn, L->w_rows[3], (int64_t)c->n_heads * vd, m->proj, th);
        for (int64_t i = 0; i < dim; i++) m->x[i] += m->proj[i];
        orc_rms_norm(m->x, L->ffn_norm, c->eps, dim, m->xn);
        orc_matvec((int)L->w_type[4], L->w[4], m->xn, L->w_rows[4], dim, m->gate, th);
        orc_matvec((int)L->w_type[5], L->w[5], m->xn, L->w_rows[5], dim, m->up, th);
        orc_silu_mul_avx2(m->gate, m->up, m->hidden, c->hidden_dim);
        orc_matvec((int)L->w_type[6], L->w[6], m->hidden, L->w_rows[6], c->hidden_dim, m->proj, th);
        for (int64_t i = 0; i < dim; i++) m->x[i] += m->proj[i];
    }
    if (!want_logits) return;
    orc_rms_norm(m->x, m->output_norm, c->eps, dim, m->xn);
    orc_matvec((int)m->output_type, m->output_w, m->xn, c->vocab, dim, logits, th);
}

void orc_model_forward(orc_model *m, uint32_t token, int64_t pos, float *logits, int want_logits) {
    orc_model_forward_from(m, token, pos, -1, logits, want_logits);
}

int64_t orc_model_generate(orc_model *m, const uint32_t *prompt, int64_t n_prompt, int64_t start_pos, int64_t n_gen,
                           float penalty, uint32_t *out_tokens, float *last_logits) {
    int64_t vocab = m->c.vocab;
    float *logits = (float *)malloc((size_t)vocab * 4);
    uint32_t recent[64];
    int64_t nrecent = 0;
    /* recent_token_tail of the prompt (runtime.rs:508-512) */
    int64_t tail = n_prompt > 64 ? n_prompt - 64 : 0;
    for (int64_t i = tail; i < n_prompt; i++) recent[nrecent++] = prompt[i];
    int64_t pos = start_pos;
    for (int64_t i = 0; i < n_prompt; i++, pos++)
        orc_model_forward(m, prompt[i], pos, logits, i + 1 == n_prompt);
    int64_t produced = 0;
    for (int64_t g = 0; g < n_gen; g++) {
        /* report the forward's logits, not the penalised copy the sampler edits */
        if (last_logits) memcpy(last_logits, logits, (size_t)vocab * 4);
        uint32_t tok = orc_greedy(logits, vocab, recent, nrecent, penalty);
        out_tokens[produced++] = tok;
        /* push_recent_token, runtime.rs:514-521 */
        if (nrecent == 64) {
            memmove(recent, recent + 1, 63 * sizeof(uint32_t));
            recent[63] = tok;
        } else {
            recent[nrecent++] = tok;
        }
        if (g + 1 == n_gen) break;
        orc_model_forward(m, tok, pos, logits, 1);
        pos++;
    }
    if (last_logits && n_gen == 0) memcpy(last_logits, logits, (size_t)vocab * 4);
    free(logits);
    return produced;
}

/* ------------------------------------------------------------------------ */
/* gpt-oss decode model: forward_gpt_oss_into, model.rs:6733-6908 (and, with
 * want_logits = 0, forward_prefill_gpt_oss = forward_hidden_gpt_oss_impl
 * without the final norm, model.rs:10286-10295: the same layer loop, no
 * head), with the reference's KVCache::with_sliding_window(max_len, window)
 * (model.rs:1363-1385): a window > 0 makes every layer's cache a ring of
 * storage_len_for(max_len, window) = min(window, max_len) slots, position p
 * at slot p % storage (slot_for_pos, :1458-1464), and every layer's attention
 * scans that ring with slot_count = storage (:6793-6810); even layers start
 * at attention_start_pos(pos, window), odd layers at 0.                      */
struct orc_gptoss {
    orc_gptoss_config c;
    orc_gptoss_layer *layers;
    const float *output_norm;
    const uint8_t *output_w, *embd;
    uint32_t output_type, embd_type;
    float *inv_freq;
    int64_t storage;
    float **k, **v;
    float *x, *xn, *xn2, *q, *kk, *vv, *attn, *proj, *router, *gate, *up, *moe;
};

orc_gptoss *orc_gptoss_create(const orc_gptoss_config *cfg) {
    orc_gptoss *m = (orc_gptoss *)calloc(1, sizeof(orc_gptoss));
    m->c = *cfg;
    int64_t max_len = cfg->max_len > 0 ? cfg->max_len : 1;
    m->storage = cfg->sliding_window > 0 ? (cfg->sliding_window < max_len ? cfg->sliding_window : max_len) : max_len;
    int64_t kdim = (int64_t)cfg->n_kv_heads * cfg->head_dim, vdim = (int64_t)cfg->n_kv_heads * cfg->value_dim;
    m->layers = (orc_gptoss_layer *)calloc((size_t)cfg->n_layers, sizeof(orc_gptoss_layer));
    m->k = (float **)calloc((size_t)cfg->n_layers, sizeof(float *));
    m->v = (float **)calloc((size_t)cfg->n_layers, sizeof(float *));
    for (int l = 0; l < cfg->n_layers; l++) {
        m->k[l] = (float *)calloc((size_t)(m->storage * kdim), 4);
        m->v[l] = (float *)calloc((size_t)(m->storage * vdim), 4);
    }
    int64_t dim = cfg->dim, hid = cfg->hidden_dim;
    m->x = (float *)calloc((size_t)dim, 4);
    m->xn = (float *)calloc((size_t)dim, 4);
    m->xn2 = (float *)calloc((size_t)dim, 4);
    m->q = (float *)calloc((size_t)cfg->n_heads * cfg->head_dim, 4);
    m->kk = (float *)calloc((size_t)kdim, 4);
    m->vv = (float *)calloc((size_t)vdim, 4);
    m->attn = (float *)calloc((size_t)cfg->n_heads * cfg->value_dim, 4);
    m->proj = (float *)calloc((size_t)dim, 4);
    m->router = (float *)calloc((size_t)cfg->n_experts, 4);
    m->gate = (float *)calloc((size_t)hid, 4);
    m->up = (float *)calloc((size_t)hid, 4);
    m->moe = (float *)calloc((size_t)dim, 4);
    m->inv_freq = (float *)calloc((size_t)cfg->head_dim, 4);
    return m;
}

void orc_gptoss_free(orc_gptoss *m) {
    if (!m) return;
    for (int l = 0; l < m->c.n_layers; l++) {
        free(m->k[l]);
        free(m->v[l]);
    }
    free(m->k); free(m->v); free(m->layers);
    free(m->x); free(m->xn); free(m->xn2); free(m->q); free(m->kk); free(m->vv); free(m->attn);
    free(m->proj); free(m->router); free(m->gate); free(m->up); free(m->moe); free(m->inv_freq);
    free(m);
}

int orc_gptoss_set_layer(orc_gptoss *m, int32_t l, const orc_gptoss_layer *layer) {
    if (l < 0 || l >= m->c.n_layers) return 0;
    m->layers[l] = *layer;
    return 1;
}

int orc_gptoss_set_output(orc_gptoss *m, const float *output_norm, const uint8_t *output_w, uint32_t output_type,
                          const uint8_t *embd, uint32_t embd_type, const float *inv_freq) {
    m->output_norm = output_norm;
    m->output_w = output_w;
    m->output_type = output_type;
    m->embd = embd;
    m->embd_type = embd_type;
    memcpy(m->inv_freq, inv_freq, (size_t)(m->c.head_dim / 2) * 4);
    return 1;
}

int64_t orc_gptoss_storage(const orc_gptoss *m) { return m->storage; }
float *orc_gptoss_kv(orc_gptoss *m, int32_t layer, int32_t which) { return which ? m->v[layer] : m->k[layer]; }

void orc_gptoss_forward(orc_gptoss *m, uint32_t token, int64_t pos, float *logits, int want_logits) {
    const orc_gptoss_config *c = &m->c;
    const int64_t dim = c->dim, hd = c->head_dim, vd = c->value_dim, nh = c->n_heads, nkv = c->n_kv_heads;
    const int64_t hid = c->hidden_dim, kdim = nkv * hd, vdim = nkv * vd, kv_mul = nh / nkv;
    const int th = g_threads;
    orc_dequant_row((int)m->embd_type, m->embd + (int64_t)token * orc_row_bytes((int)m->embd_type, dim), m->x, dim);
    const int64_t slot = c->sliding_window > 0 ? pos % m->storage : pos;
    const float scale = 1.0f / sqrtf((float)hd);
    for (int l = 0; l < c->n_layers; l++) {
        const orc_gptoss_layer *L = &m->layers[l];
        orc_rms_norm(m->x, L->attn_norm, c->eps, dim, m->xn);
        orc_matvec((int)L->wq_type, L->wq, m->xn, nh * hd, dim, m->q, th);
        orc_matvec((int)L->wk_type, L->wk, m->xn, kdim, dim, m->kk, th);
        orc_matvec((int)L->wv_type, L->wv, m->xn, vdim, dim, m->vv, th);
        for (int64_t i = 0; i < nh * hd; i++) m->q[i] += L->bq[i];
        for (int64_t i = 0; i < kdim; i++) m->kk[i] += L->bk[i];
        for (int64_t i = 0; i < vdim; i++) m->vv[i] += L->bv[i];
        orc_rope_gpt_oss(m->q, m->kk, pos, hd, nh, nkv, c->concentration, m->inv_freq);
        memcpy(m->k[l] + slot * kdim, m->kk, (size_t)kdim * 4);
        memcpy(m->v[l] + slot * vdim, m->vv, (size_t)vdim * 4);
        const int64_t start = l % 2 == 0 ? orc_attention_start_pos(pos, c->sliding_window) : 0;
        orc_attention_sink_heads(m->q, m->k[l], m->v[l], L->sinks, kdim, vdim, m->storage, hd, vd, nh, kv_mul, start,
                                 pos, scale, m->attn);
        orc_matvec((int)L->wo_type, L->wo, m->attn, dim, nh * vd, m->proj, th);
        for (int64_t i = 0; i < dim; i++) m->x[i] += m->proj[i] + L->bo[i];
        orc_rms_norm(m->x, L->post_attn_norm, c->eps, dim, m->xn2);
        /* router: gate_inp + bias, top-k in total order, softmax over the
         * chosen (model.rs:6846-6857) */
        orc_matvec((int)L->router_type, L->router, m->xn2, c->n_experts, dim, m->router, th);
        for (int64_t i = 0; i < c->n_experts; i++) m->router[i] += L->router_bias[i];
        int32_t sel[64];
        float val[64], prob[64];
        orc_select_top_logits(m->router, c->n_experts, c->top_k, sel, val);
        orc_softmax_selected(val, c->top_k, prob);
        const int64_t rg = orc_row_bytes((int)L->exps_type, dim) * hid;
        const int64_t rd = orc_row_bytes((int)L->exps_type, hid) * dim;
        memset(m->moe, 0, (size_t)dim * 4);
        for (int64_t s = 0; s < c->top_k; s++) {
            const int64_t e = sel[s];
            const float *gb = L->gate_exps_bias + e * hid, *ub = L->up_exps_bias + e * hid;
            const float *db = L->down_exps_bias + e * dim;
            orc_matvec((int)L->exps_type, L->gate_exps + e * rg, m->xn2, hid, dim, m->gate, th);
            orc_matvec((int)L->exps_type, L->up_exps + e * rg, m->xn2, hid, dim, m->up, th);
            for (int64_t i = 0; i < hid; i++) m->gate[i] = orc_swiglu_gpt_oss(m->gate[i] + gb[i], m->up[i] + ub[i]);
            orc_matvec((int)L->exps_type, L->down_exps + e * rd, m->gate, dim, hid, m->proj, th);
            for (int64_t i = 0; i < dim; i++) m->moe[i] += (m->proj[i] + db[i]) * prob[s];
        }
        for (int64_t i = 0; i < dim; i++) m->x[i] += m->moe[i];
    }
    if (!want_logits) return;
    orc_rms_norm(m->x, m->output_norm, c->eps, dim, m->xn);
    orc_matvec((int)m->output_type, m->output_w, m->xn, c->vocab, dim, logits, th);
}

/* ------------------------------------------------------------------------ */
/* Reference test fixtures (byte generators from src/simd.rs tests).         */
void orc_make_q4k_weights(int64_t rows, int64_t cols, uint8_t seed, uint8_t *data) {
    /* simd.rs:7661-7682 */
    int64_t rb = (cols / 256) * 144;
    for (int64_t row = 0; row < rows; row++)
        for (int64_t block = 0; block < cols / 256; block++) {
            uint8_t *base = data + row * rb + block * 144;
            base[0] = 0x00; base[1] = 0x3c; base[2] = 0x00; base[3] = 0x00;
            for (int i = 0; i < 12; i++) base[4 + i] = (uint8_t)(1 + (((uint8_t)(seed + (uint8_t)row + (uint8_t)i)) & 0x07));
            for (int i = 0; i < 128; i++) base[16 + i] = (uint8_t)(seed + (uint8_t)(row * 17 + block * 29 + i * 3)) & 0x7f;
        }
}

void orc_make_q4k_weights_dmin(int64_t rows, int64_t cols, uint8_t seed, uint8_t *data) {
    /* simd.rs:8259-8279 */
    int64_t rb = (cols / 256) * 144;
    for (int64_t row = 0; row < rows; row++)
        for (int64_t block = 0; block < cols / 256; block++) {
            uint8_t *base = data + row * rb + block * 144;
            base[0] = 0x00; base[1] = 0x3c; base[2] = 0x00; base[3] = 0x38;
            for (int i = 0; i < 12; i++) base[4 + i] = (uint8_t)(seed + (uint8_t)(row * 5 + block * 7 + i * 11));
            for (int i = 0; i < 128; i++) base[16 + i] = (uint8_t)(seed + (uint8_t)(row * 17 + block * 29 + i * 3)) & 0x7f;
        }
}

void orc_make_q6k_weights(int64_t rows, int64_t cols, uint8_t seed, uint8_t *data) {
    /* simd.rs:7718-7738 */
    int64_t rb = (cols / 256) * 210;
    for (int64_t row = 0; row < rows; row++)
        for (int64_t block = 0; block < cols / 256; block++) {
            uint8_t *base = data + row * rb + block * 210;
            for (int i = 0; i < 128; i++) base[i] = (uint8_t)(seed + (uint8_t)(row * 7 + block * 13 + i * 3));
            for (int i = 0; i < 64; i++) base[128 + i] = (uint8_t)(seed + (uint8_t)(row * 11 + block * 17 + i * 5));
            for (int i = 0; i < 16; i++) base[192 + i] = (uint8_t)(1 + (((uint8_t)(seed + (uint8_t)i)) & 0x07));
            base[208] = 0x00; base[209] = 0x3c;
        }
}

void orc_make_q8_0_row_scaled(int64_t cols, uint8_t seed, uint8_t *data) {
    /* simd.rs:8665-8679 with F16_SCALES of simd.rs:8629 */
    static const uint16_t F16_SCALES[6] = {0x3C00, 0x3800, 0x3400, 0x3E00, 0x4000, 0xB800};
    for (int64_t b = 0; b < cols / 32; b++) {
        uint8_t *base = data + b * 34;
        uint16_t s = F16_SCALES[(b + seed) % 6];
        base[0] = (uint8_t)(s & 0xff);
        base[1] = (uint8_t)(s >> 8);
        for (int i = 0; i < 32; i++) base[2 + i] = (uint8_t)(seed + (uint8_t)(b * 13 + i * 7));
    }
}

void orc_make_mxfp4_test_row(int64_t blocks, uint8_t *row) {
    /* simd.rs:7836-7846 */
    for (int64_t block = 0; block < blocks; block++) {
        uint8_t *base = row + block * 17;
        for (int i = 0; i < 16; i++) {
            uint8_t lo = (uint8_t)((block * 7 + i * 3 + 1) & 0x0f);
            uint8_t hi = (uint8_t)((block * 11 + i * 5 + 9) & 0x0f);
            base[i] = (uint8_t)(lo | (hi << 4));
        }
        base[16] = (uint8_t)(123 + (uint8_t)(block % 9));
    }
}

void orc_test_activation(int64_t cols, float *out) {
    /* simd.rs:8685-8689 */
    for (int64_t i = 0; i < cols; i++) out[i] = (sinf((float)i * 0.017f) * 0.45f) - ((float)(i % 7) * 0.021f);
}

void orc_mxfp4_test_activation(int64_t n, float *out) {
    /* simd.rs:7847-7849 */
    for (int64_t i = 0; i < n; i++) out[i] = sinf((float)i * 0.071f) * 0.9f + (float)(i % 13) * 0.02f;
}

/* libm expf over an array: exp_attn (model.rs:5720-5726) is f32::exp. */
void orc_expf_array(const float *x, int64_t n, float *out) {
    for (int64_t i = 0; i < n; i++) out[i] = expf(x[i]);
}
