// attention_exact.hip — GQA decode attention that reproduces the reference's
// online softmax (src/model.rs:5739-6198) bit for bit.
//
// The reference scans positions start_t..=end_t serially per query head:
//   score = dot(q, k) * scale
//   if score > max: old = isfinite(max) ? expf(max - score) : 0
//                   out = out*old + v   (one fused rounding or two, by path)
//                   denom = denom*old + 1;  max = score
//   else:           w = expf(score - max);  out += w*v (fused);  denom += w
//   out *= 1/denom
// Only the out/denom recurrences are inherently serial.  The work is split so
// everything else runs in parallel and the serial part is one FMA per step:
//   A  attn_exact_scores:  scores with the reference's dot-product lane order
//      (dot_f32x4_avx2 for the first four heads of a kv_mul 4/6 group,
//      dot_f32_avx2 otherwise), all positions in parallel.
//   B  attn_exact_coef:    per head, an exact prefix-max scan gives the running
//      max before every step, so each step's branch and expf argument are
//      known up front; expf is glibc's (restated below, checked against
//      glibc on all 2^32 inputs).
//   C  attn_exact_chain:   one wave per (query head, 64 value dims) runs the
//      FMA recurrence with a wave-uniform branch; an extra wave runs the
//      denominators; out = out * (1/denom).
// Which update form a head uses follows the reference: affine_add_f32x4
// (fma(v, alpha, out*mul)) for heads 0..3 of kv_mul 4/6 groups, scale_add /
// axpy (fma(out, old, v) / fma(w, v, out)) otherwise; with sinks every head
// uses the per-head sink scan (online_attention_with_sink).
#include "common.hpp"

namespace rh {

// ---- expf of glibc 2.35 on x86-64 with FMA ------------------------------------
// The published ARM optimized-routines expf that glibc uses: x*N/ln2 = k + r,
// exp(x) = 2^(k/N) * 2^(r/N), N = 32, 2^(k/N) from a 32-entry table
// (tab[i] = bits(2^(i/32)) - (i << 47)), 2^(r/N) from a cubic, all in double.
// The fused multiply-adds are where GCC contracts them in glibc's FMA build.
__constant__ uint64_t kExp2fTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

__device__ __forceinline__ float expf_glibc(float x) {
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= (0x42b00000u >> 20)) {  // |x| >= 88 or nan
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= (0x7f800000u >> 20)) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_bit_cast(float, 0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double invln2n = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32768.0, c1 = 0x1.ebfce50fac4f3p-3 / 1024.0,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    double xd = (double)x;
    double kd = __builtin_fma(invln2n, xd, shift);
    uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    double r = __builtin_fma(invln2n, xd, -kd);
    uint64_t t = kExp2fTab[ki % 32] + (ki << 47);
    double s = __builtin_bit_cast(double, t);
    double z = __builtin_fma(c0, r, c1);
    double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

struct AttnExactArgs {
    const float *q;      // [n_heads * hd]
    const float *k;      // cache base, slot s, kv head h at k + s*key_stride + h*hd
    const float *v;
    const float *sinks;  // [n_heads] or null
    float *scores;       // [n_heads][cap]
    float2 *coef;        // [n_heads][cap]: (e, new-max flag)
    uint32_t *newmask;   // [n_heads][cap/32]: bit t%32 set when step t sets a new max
    float *out;          // [n_heads * vd]
    const StepState *st;
    int32_t n_heads, n_kv, kv_mul, hd, vd;
    int64_t key_stride, value_stride;
    int32_t slot_count, start_t, end_t, window, cap;
    float scale;
};

__device__ __forceinline__ void exact_range(const AttnExactArgs &A, int &s, int &e) {
    if (A.st) {
        e = A.st->pos;
        s = A.window > 0 ? max(0, e + 1 - A.window) : A.st->start_t;
    } else {
        s = A.start_t;
        e = A.end_t;
    }
}

// heads 0..3 of a kv_mul 4/6 group take the x4 path (online_attention_grouped,
// src/model.rs:6089-6125); sinks force the per-head scan.
__device__ __forceinline__ bool is_x4(const AttnExactArgs &A, int g) {
    return A.sinks == nullptr && (A.kv_mul == 4 || A.kv_mul == 6) && g < 4;
}

#define EX_TILE 64

// A: one workgroup per (tile of EX_TILE positions, kv head).
__global__ __launch_bounds__(256) void attn_exact_scores_kernel(AttnExactArgs A) {
    extern __shared__ float s_dyn[];
    const int hd = A.hd, kvm = A.kv_mul;
    const int ldk = hd + 1;  // padded row: no bank conflicts on column reads
    float *s_q = s_dyn;               // [kv_mul][hd]
    float *s_k = s_dyn + kvm * hd;    // [EX_TILE][hd+1]
    int s0, e0;
    exact_range(A, s0, e0);
    const int ctx = e0 - s0 + 1;
    const int t_base = blockIdx.x * EX_TILE;
    if (ctx <= 0 || t_base >= ctx) return;
    const int h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nt = min(EX_TILE, ctx - t_base);
    for (int i = tid; i < kvm * hd; i += 256) s_q[i] = A.q[(size_t)h * kvm * hd + i];
    for (int i = tid; i < nt * hd; i += 256) {
        int tt = i / hd, c = i % hd;
        int slot = (s0 + t_base + tt) % A.slot_count;
        s_k[tt * ldk + c] = A.k[(size_t)slot * A.key_stride + (size_t)h * hd + c];
    }
    __syncthreads();
    // x4 heads: 8 lanes per (head, position), one accumulator per lane,
    // chained over the hd/8 chunks, then hsum_avx.
    const int nx4 = (A.sinks == nullptr && (kvm == 4 || kvm == 6)) ? 4 : 0;
    {
        const int pairs = nx4 * nt;
        const int l = lane & 7;
        for (int p0 = wave * 8; p0 < ((pairs + 7) / 8) * 8; p0 += 32) {
            int p = p0 + (lane >> 3);
            bool ok = p < pairs;
            int g = ok ? p / nt : 0, tt = ok ? p % nt : 0;
            float s = 0.0f;
            if (ok) {
                const float *qq = s_q + g * hd, *kk = s_k + tt * ldk;
                for (int c = 0; c + 8 <= hd; c += 8) s = fmaf(qq[c + l], kk[c + l], s);
            }
            float a = s + __shfl_xor(s, 4, 64);
            float b = a + __shfl_xor(a, 1, 64);
            float d = b + __shfl_xor(b, 2, 64);
            if (ok && l == 0) {
                const float *qq = s_q + g * hd, *kk = s_k + tt * ldk;
                for (int c = hd - hd % 8; c < hd; c++) d += qq[c] * kk[c];
                A.scores[(size_t)(h * kvm + g) * A.cap + t_base + tt] = d * A.scale;
            }
        }
    }
    // other heads: dot_f32_avx2 (src/simd.rs:6547-6586): 32 lanes = four
    // 8-wide accumulators over 32-element chunks, (a0+a1)+(a2+a3), the 8-chunk
    // tail, hsum_avx, then the scalar tail.
    {
        const int ng = kvm - nx4;
        const int pairs = ng * nt;
        const int L = lane & 31;
        const int main32 = hd / 32, tail8 = (hd - main32 * 32) / 8;
        for (int p0 = wave * 2; p0 < ((pairs + 1) / 2) * 2; p0 += 8) {
            int p = p0 + (lane >> 5);
            bool ok = p < pairs;
            int g = ok ? nx4 + p / nt : 0, tt = ok ? p % nt : 0;
            const float *qq = s_q + g * hd, *kk = s_k + tt * ldk;
            float acc = 0.0f;
            if (ok)
                for (int c = 0; c < main32; c++) acc = fmaf(qq[32 * c + L], kk[32 * c + L], acc);
            float x = acc + __shfl_xor(acc, 8, 64);   // lane l (<8): a0+a1; lane 16+l: a2+a3
            float y = x + __shfl_xor(x, 16, 64);      // lane l: (a0+a1)+(a2+a3)
            if (ok && L < 8)
                for (int i = 0; i < tail8; i++) y = fmaf(qq[32 * main32 + 8 * i + L], kk[32 * main32 + 8 * i + L], y);
            float a = y + __shfl_xor(y, 4, 64);
            float b = a + __shfl_xor(a, 1, 64);
            float d = b + __shfl_xor(b, 2, 64);
            if (ok && L == 0) {
                for (int c = 32 * main32 + 8 * tail8; c < hd; c++) d += qq[c] * kk[c];
                A.scores[(size_t)(h * kvm + g) * A.cap + t_base + tt] = d * A.scale;
            }
        }
    }
}

// B: one workgroup per query head: exact running max before each step, then
// every step's branch and expf value.
__global__ __launch_bounds__(256) void attn_exact_coef_kernel(AttnExactArgs A) {
    __shared__ float s_seg[256];
    int s0, e0;
    exact_range(A, s0, e0);
    const int ctx = e0 - s0 + 1;
    if (ctx <= 0) return;
    const int head = blockIdx.x, tid = threadIdx.x;
    const float *sc = A.scores + (size_t)head * A.cap;
    const float init = A.sinks ? A.sinks[head] : -INFINITY;
    const int per = (ctx + 255) / 256;
    const int b0 = tid * per, b1 = min(ctx, b0 + per);
    float m = -INFINITY;
    for (int t = b0; t < b1; t++) m = fmaxf(m, sc[t]);
    s_seg[tid] = m;
    __syncthreads();
    // exclusive prefix max of the segment maxima (max is exact in any order)
    for (int off = 1; off < 256; off <<= 1) {
        float o = tid >= off ? s_seg[tid - off] : -INFINITY;
        __syncthreads();
        s_seg[tid] = fmaxf(s_seg[tid], o);
        __syncthreads();
    }
    float run = fmaxf(init, tid > 0 ? s_seg[tid - 1] : -INFINITY);
    float2 *cf = A.coef + (size_t)head * A.cap;
    for (int t = b0; t < b1; t++) {
        float s = sc[t];
        float2 c;
        if (s > run) {
            c.x = __builtin_isfinite(run) ? expf_glibc(run - s) : 0.0f;
            c.y = 1.0f;
            run = s;
        } else {
            c.x = expf_glibc(s - run);
            c.y = 0.0f;
        }
        cf[t] = c;
    }
    __syncthreads();
    // bit masks of new-max steps, 32 positions per word
    uint32_t *mk = A.newmask + (size_t)head * (A.cap / 32);
    for (int w = tid; w < (ctx + 31) / 32; w += 256) {
        uint32_t bits = 0;
        for (int j = 0; j < 32; j++) {
            int t = w * 32 + j;
            if (t < ctx && cf[t].y != 0.0f) bits |= 1u << j;
        }
        mk[w] = bits;
    }
}

// C: one wave per (query head, 64 value dims), grid (n_heads, ceil(vd/64)).
// Each lane runs the output recurrence of one dim; the denominator recurrence
// is wave-uniform and runs alongside in every lane (an independent chain, so
// it costs no extra latency).  Coefficients are prefetched 32 steps at a time.
__global__ __launch_bounds__(64) void attn_exact_chain_kernel(AttnExactArgs A) {
    int s0, e0;
    exact_range(A, s0, e0);
    const int ctx = e0 - s0 + 1;
    if (ctx <= 0) return;
    const int head = blockIdx.x, slice = blockIdx.y, lane = threadIdx.x;
    const int kvm = A.kv_mul, h = head / kvm, g = head % kvm;
    const int dim = slice * 64 + lane;
    const bool dim_ok = dim < A.vd;
    const bool x4 = is_x4(A, g);
    const float2 *cf = A.coef + (size_t)head * A.cap;
    const uint32_t *mk = A.newmask + (size_t)head * (A.cap / 32);
    const float *vbase = A.v + (size_t)h * A.vd + (dim_ok ? dim : 0);
    float o = 0.0f;
    float d = A.sinks ? 1.0f : 0.0f;
    for (int t0 = 0; t0 < ctx; t0 += 32) {
        const int n = min(32, ctx - t0);
        float vb[32];
        float2 cb[32];
#pragma unroll
        for (int j = 0; j < 32; j++) {
            int t = t0 + j < ctx ? t0 + j : ctx - 1;
            int slot = (s0 + t) % A.slot_count;
            vb[j] = vbase[(size_t)slot * A.value_stride];
            cb[j] = cf[t];
        }
        const uint32_t bits = mk[t0 >> 5];
        if (bits == 0 && n == 32) {
#pragma unroll
            for (int j = 0; j < 32; j++) {
                o = fmaf(cb[j].x, vb[j], o);
                d = d + cb[j].x;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 32; j++) {
                if (j < n) {
                    if (cb[j].y != 0.0f) {
                        if (x4)
                            o = fmaf(vb[j], 1.0f, o * cb[j].x);  // affine_add: fma(value, 1, out*old)
                        else
                            o = fmaf(o, cb[j].x, vb[j]);         // scale_add: fma(out, old, value)
                        float p = d * cb[j].x;
                        d = p + 1.0f;
                    } else {
                        o = fmaf(cb[j].x, vb[j], o);             // axpy / affine_add with mul 1
                        d = d + cb[j].x;
                    }
                }
            }
        }
    }
    if (dim_ok) {
        float r = o;
        if (d > 0.0f) {
            float inv = 1.0f / d;
            r = o * inv;
        }
        A.out[(size_t)head * A.vd + dim] = r;
    }
}

}  // namespace rh
