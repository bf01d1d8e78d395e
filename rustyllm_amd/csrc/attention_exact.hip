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
//   B  attn_exact_coef:    per (64-position tile, head), the running max
//      before every step from the tile maxima and an in-tile prefix max, so
//      each step's branch and expf argument are known up front; expf is
//      glibc's (restated below, checked against glibc on all 2^32 inputs).
//   C  attn_exact_chain:   the FMA recurrences, one lane per (head, dim),
//      V streamed into LDS by direct global->LDS loads; the denominators run
//      as the same recurrence with v = 1.
//   D  attn_exact_finish:  out = out * (1/denom), fused with the Q8_K
//      quantization the output projection needs.
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
    float *scores;       // [n_heads][cap]   q.k * scale per position
    float *e;            // [n_kv][ceil(kv_mul/4)][cap][4]  the step's expf value
                         // (see below), four heads of a kv group interleaved
    float *tmax;         // [n_heads][cap/64] max score of each 64-position tile
    uint32_t *newmask;   // [n_heads][cap/32] bit t%32 set when step t sets a new max
    float *den;          // [n_heads]         final denominators
    float *out;          // [n_heads * vd]    un-normalised outputs
    const StepState *st;
    int32_t n_heads, n_kv, kv_mul, hd, vd;
    int64_t key_stride, value_stride;
    int32_t slot_count, start_t, end_t, window, cap;
    int32_t kvec;        // 1: K rows are 16-byte aligned (float4 loads)
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

// e of (kv head h, head g of its group, position t): groups of four heads are
// interleaved per position so one 64-position tile of a group is 1 KB.
__device__ __forceinline__ size_t e_index(const AttnExactArgs &A, int h, int g, int t) {
    const int hgroups = (A.kv_mul + 3) / 4;
    return ((size_t)(h * hgroups + g / 4) * A.cap + t) * 4 + (g & 3);
}

// A: one workgroup per (tile of EX_TILE positions, kv head).  Writes the
// scores of every query head of the group and each head's tile maximum.
__global__ __launch_bounds__(256) void attn_exact_scores_kernel(AttnExactArgs A) {
    extern __shared__ float s_dyn[];
    const int hd = A.hd, kvm = A.kv_mul;
    const int ldk = hd + 1;  // padded row: no bank conflicts on column reads
    float *s_q = s_dyn;                       // [kv_mul][hd]
    float *s_k = s_q + kvm * hd;              // [EX_TILE][hd+1]
    float *s_sc = s_k + EX_TILE * ldk;        // [kv_mul][EX_TILE]
    int s0, e0;
    exact_range(A, s0, e0);
    const int ctx = e0 - s0 + 1;
    const int t_base = blockIdx.x * EX_TILE;
    if (ctx <= 0 || t_base >= ctx) return;
    const int h = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nt = min(EX_TILE, ctx - t_base);
    for (int i = tid; i < kvm * hd; i += 256) s_q[i] = A.q[(size_t)h * kvm * hd + i];
    const float *kh = A.k + (size_t)h * hd;
    if (A.kvec) {
        const int h4 = hd >> 2;
#pragma unroll 8
        for (int i = tid; i < nt * h4; i += 256) {
            int tt = i / h4, c = (i - tt * h4) * 4;
            int slot = (s0 + t_base + tt) % A.slot_count;
            float4 v = *(const float4 *)(kh + (size_t)slot * A.key_stride + c);
            float *d = s_k + tt * ldk + c;
            d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
        }
    } else {
#pragma unroll 4
        for (int i = tid; i < nt * hd; i += 256) {
            int tt = i / hd, c = i - tt * hd;
            int slot = (s0 + t_base + tt) % A.slot_count;
            s_k[tt * ldk + c] = kh[(size_t)slot * A.key_stride + c];
        }
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
                s_sc[g * EX_TILE + tt] = d * A.scale;
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
                s_sc[g * EX_TILE + tt] = d * A.scale;
            }
        }
    }
    __syncthreads();
    // coalesced score rows + tile maxima (max is exact in any order)
    const int ntl = A.cap / EX_TILE;
    for (int g = wave; g < kvm; g += 4) {
        const int head = h * kvm + g;
        float v = lane < nt ? s_sc[g * EX_TILE + lane] : -INFINITY;
        if (lane < nt) A.scores[(size_t)head * A.cap + t_base + lane] = v;
        float m = wave_max(v);
        if (lane == 0) A.tmax[(size_t)head * ntl + blockIdx.x] = m;
    }
}

// B: one wave per (tile of 64 positions, query head).  The running max before
// each step is max(initial, maxima of the earlier tiles, prefix max inside the
// tile), so every step's branch and expf argument are known without a serial
// scan.  e[t] = isfinite(run) ? expf(run - s) : 0 on a new max (the factor the
// old output and denominator are scaled by), expf(s - run) otherwise; the
// new-max steps are marked in newmask.
__global__ __launch_bounds__(64) void attn_exact_coef_kernel(AttnExactArgs A) {
    int s0, e0;
    exact_range(A, s0, e0);
    const int ctx = e0 - s0 + 1;
    const int tile = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
    if (ctx <= 0 || tile * EX_TILE >= ctx) return;
    const int ntl = A.cap / EX_TILE;
    const float *tm = A.tmax + (size_t)head * ntl;
    float m = -INFINITY;
    for (int j = lane; j < tile; j += 64) m = fmaxf(m, tm[j]);
    m = wave_max(m);
    if (A.sinks) m = fmaxf(A.sinks[head], m);
    const int t = tile * EX_TILE + lane;
    const bool valid = t < ctx;
    const float s = valid ? A.scores[(size_t)head * A.cap + t] : -INFINITY;
    float p = s;  // inclusive prefix max over lanes
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        float q = __shfl_up(p, o, 64);
        if (lane >= o) p = fmaxf(p, q);
    }
    float prev = __shfl_up(p, 1, 64);
    const float run = lane == 0 ? m : fmaxf(m, prev);
    const bool flag = valid && s > run;
    float e = 0.0f;
    if (flag)
        e = __builtin_isfinite(run) ? expf_glibc(run - s) : 0.0f;
    else if (valid)
        e = expf_glibc(s - run);
    const int kvm = A.kv_mul, g = head % kvm;
    A.e[e_index(A, head / kvm, g, t)] = e;
    const unsigned long long bits = __ballot(flag);
    if (lane < 2) A.newmask[(size_t)head * (A.cap / 32) + 2 * tile + lane] = (uint32_t)(bits >> (32 * lane));
}

// C: the output and denominator recurrences
//   new max: out = affine_add: fma(v, 1, out*e) | scale_add: fma(out, e, v)
//            den = den*e + 1 (two roundings)
//   else:    out = fma(e, v, out);  den = den + e
// in the reference's step order.  One wave covers up to four query heads of a
// kv group (lane = head slot * 16 + dim) for 16 value dims, so every V element
// is read from HBM once per layer.  An extra "slice" per group runs the
// denominator as the same recurrence with v = 1 (fma(e, 1, d) = d + e and
// fma(1, 1, d*e) = d*e + 1 round exactly like the reference's scalar ops).
//
// V, e and the new-max words reach LDS through direct global->LDS loads
// (global_load_lds_dwordx4 / _dword) into a ring of CH_NT 64-position tiles,
// CH_P tiles ahead of the recurrence; the wave waits on its own vmcnt, so no
// barrier is involved.  LDS is read only with 32-bit reads (ds_read_b32 /
// ds_read2_b32): the compiler drains vmcnt to zero before any wider LDS read
// while direct loads are in flight, which would empty the pipeline.
#ifndef CH_NT
#define CH_NT 16
#endif
#ifndef CH_P
#define CH_P 11
#endif
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ void dma16(const void *src, void *lds) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t *)lds, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void *src, void *lds) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t *)lds, 4, 0, 0);
}

// s_waitcnt vmcnt(N) with expcnt/lgkmcnt left at their maxima (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14).
#define RH_WAIT_VM(N) __builtin_amdgcn_s_waitcnt(((N) & 15) | (((N) >> 4) << 14) | (7 << 4) | (15 << 8))

template <int IPT>
__device__ __forceinline__ void wait_tiles_after(int n_after) {
    // n_after: tiles issued after the one about to be read (0..CH_P-1)
    switch (n_after) {
        case 10: RH_WAIT_VM(10 * IPT); break;
        case 9: RH_WAIT_VM(9 * IPT); break;
        case 8: RH_WAIT_VM(8 * IPT); break;
        case 7: RH_WAIT_VM(7 * IPT); break;
        case 6: RH_WAIT_VM(6 * IPT); break;
        case 5: RH_WAIT_VM(5 * IPT); break;
        case 4: RH_WAIT_VM(4 * IPT); break;
        case 3: RH_WAIT_VM(3 * IPT); break;
        case 2: RH_WAIT_VM(2 * IPT); break;
        case 1: RH_WAIT_VM(1 * IPT); break;
        default: RH_WAIT_VM(0); break;
    }
}
static_assert(CH_P - 1 <= 10, "wait_tiles_after covers at most 10 tiles");
static_assert(6 * (CH_P - 1) <= 63, "vmcnt is 6 bits");

struct ChainLds {
    float v[CH_NT][EX_TILE * 16];   // [slot][position][16 dims]
    float e[CH_NT][EX_TILE * 4];    // [slot][position][head slot]
    uint32_t m[CH_NT][8];           // [slot][head slot][2 words]
};

// 16 steps of e (position-major, stride 4 floats) and v (stride 16 floats)
template <bool DEN>
__device__ __forceinline__ void chain_load16(const float *et, const float *vt, int k, float *e, float *v) {
#pragma unroll
    for (int j = 0; j < 16; j++) {
        e[j] = et[(k * 16 + j) * 4];
        if (!DEN) v[j] = vt[(k * 16 + j) * 16];
    }
}
// 16 recurrence steps; bits = this lane's new-max flags for them.  The
// branch is wave-uniform: plain FMAs unless some head has a new max here.
template <bool DEN, bool X4>
__device__ __forceinline__ void chain_steps16(const float *e, const float *v, float &o, uint32_t bits) {
    if (!__any(bits != 0u)) {
#pragma unroll
        for (int j = 0; j < 16; j++) o = fmaf(e[j], DEN ? 1.0f : v[j], o);
    } else {
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const float vj = DEN ? 1.0f : v[j];
            const float on = fmaf(e[j], vj, o);
            const float ox = (DEN || X4) ? fmaf(vj, 1.0f, o * e[j]) : fmaf(o, e[j], vj);
            o = ((bits >> j) & 1u) ? ox : on;
        }
    }
}

template <bool DEN, bool X4>
__device__ void chain_run(const AttnExactArgs &A, ChainLds &L, int s0, int ctx, int h, int hg, int slice) {
    const int lane = threadIdx.x, gs = lane >> 4, c = lane & 15;
    const int kvm = A.kv_mul;
    const int head_g = hg * 4 + gs;
    const bool hvalid = head_g < kvm;
    const int ntiles = (ctx + EX_TILE - 1) / EX_TILE;
    constexpr int IPT = DEN ? 2 : 6;
    // DMA sources: wave-uniform bases plus 32-bit per-lane byte offsets.  V
    // row offsets advance 64 positions per tile and wrap at slot_count
    // (>= 64, so one conditional subtraction keeps them in range).
    const char *e_base = (const char *)(A.e + e_index(A, h, hg * 4, 0)) + lane * 16;
    const int m_gs = (lane >> 1) & 3;
    const int m_head = h * kvm + ((hg * 4 + m_gs < kvm) ? hg * 4 + m_gs : hg * 4);
    const char *m_base = (const char *)(A.newmask + (size_t)m_head * (A.cap / 32)) + (lane & 1) * 4;
    const char *v_base = (const char *)(A.v + (size_t)h * A.vd + slice * 16) + (lane & 3) * 16;
    const uint32_t row_bytes = (uint32_t)A.value_stride * 4u;
    const uint32_t wrap = (uint32_t)A.slot_count * row_bytes;
    const uint32_t step = 64u * row_bytes;
    uint32_t roff[4];
#pragma unroll
    for (int k = 0; k < 4; k++) roff[k] = (uint32_t)((s0 + k * 16 + (lane >> 2)) % A.slot_count) * row_bytes;

    auto issue = [&](int i) {
        const int sl = i & (CH_NT - 1);
        if (!DEN) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                dma16(v_base + roff[k], &L.v[sl][k * 256]);
                roff[k] += step;
                if (roff[k] >= wrap) roff[k] -= wrap;
            }
        }
        dma16(e_base + (uint32_t)i * 1024u, &L.e[sl][0]);
        if (lane < 8) dma4(m_base + (uint32_t)i * 8u, &L.m[sl][0]);
    };

    float o = (DEN && A.sinks) ? 1.0f : 0.0f;
    auto process = [&](int i) {
        const int sl = i & (CH_NT - 1);
        const int ntok = min(EX_TILE, ctx - i * EX_TILE);
        const float *vt = &L.v[sl][c];
        const float *et = &L.e[sl][gs];
        const uint32_t mw0 = hvalid ? L.m[sl][gs * 2] : 0u;
        const uint32_t mw1 = hvalid ? L.m[sl][gs * 2 + 1] : 0u;
        if (ntok == EX_TILE) {
            // 64 steps in 16-step chunks; LDS reads run two chunks ahead of
            // the arithmetic
            float e0[16], v0[16], e1[16], v1[16], e2[16], v2[16];
            chain_load16<DEN>(et, vt, 0, e0, v0);
            chain_load16<DEN>(et, vt, 1, e1, v1);
            chain_load16<DEN>(et, vt, 2, e2, v2);
            __builtin_amdgcn_sched_barrier(0);
            chain_steps16<DEN, X4>(e0, v0, o, mw0 & 0xFFFFu);
            __builtin_amdgcn_sched_barrier(0);
            chain_load16<DEN>(et, vt, 3, e0, v0);
            __builtin_amdgcn_sched_barrier(0);
            chain_steps16<DEN, X4>(e1, v1, o, mw0 >> 16);
            __builtin_amdgcn_sched_barrier(0);
            chain_steps16<DEN, X4>(e2, v2, o, mw1 & 0xFFFFu);
            __builtin_amdgcn_sched_barrier(0);
            chain_steps16<DEN, X4>(e0, v0, o, mw1 >> 16);
        } else {
            for (int t = 0; t < ntok; t++) {
                const uint32_t mw = t < 32 ? mw0 : mw1;
                const float e = et[t * 4];
                const float v = DEN ? 1.0f : vt[t * 16];
                const float on = fmaf(e, v, o);
                const float ox = (DEN || X4) ? fmaf(v, 1.0f, o * e) : fmaf(o, e, v);
                o = ((mw >> (t & 31)) & 1u) ? ox : on;
            }
        }
    };

    const int pro = min(CH_P - 1, ntiles);
    for (int i = 0; i < pro; i++) issue(i);
    int i = 0;
    for (; i + CH_P - 1 < ntiles; i++) {  // steady state: CH_P - 1 tiles behind this one
        issue(i + CH_P - 1);
        RH_WAIT_VM((CH_P - 1) * IPT);
        process(i);
    }
    for (; i < ntiles; i++) {  // drain
        wait_tiles_after<IPT>(ntiles - 1 - i);
        process(i);
    }
    if (hvalid) {
        const int head = h * kvm + head_g;
        if (DEN) {
            if (c == 0) A.den[head] = o;
        } else {
            A.out[(size_t)head * A.vd + slice * 16 + c] = o;
        }
    }
}

// grid: n_kv * ceil(kv_mul/4) * (vd/16 + 1) workgroups of one wave; block b
// serves kv head b % n_kv, so consecutive blocks spread over the XCDs.
__global__ __launch_bounds__(64) void attn_exact_chain_dma_kernel(AttnExactArgs A) {
    __shared__ ChainLds L;
    int s0, e0;
    exact_range(A, s0, e0);
    const int ctx = e0 - s0 + 1;
    if (ctx <= 0) return;
    const int nsl = A.vd / 16;
    const int h = blockIdx.x % A.n_kv;
    const int r = blockIdx.x / A.n_kv;
    const int hg = r / (nsl + 1), slice = r % (nsl + 1);
    if (slice == nsl) {
        chain_run<true, true>(A, L, s0, ctx, h, hg, 0);
    } else {
        const bool x4 = A.sinks == nullptr && (A.kv_mul == 4 || A.kv_mul == 6) && hg == 0;
        if (x4)
            chain_run<false, true>(A, L, s0, ctx, h, hg, slice);
        else
            chain_run<false, false>(A, L, s0, ctx, h, hg, slice);
    }
}

// C (any layout): one wave per (query head, 64 value dims), grid (n_heads,
// ceil(vd/64)); V read straight from the cache, 32 steps per batch.  The
// denominator runs in every lane beside the output; slice 0 stores it.
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
    const float *ef = A.e + e_index(A, h, g, 0);
    const uint32_t *mk = A.newmask + (size_t)head * (A.cap / 32);
    const float *vbase = A.v + (size_t)h * A.vd + (dim_ok ? dim : 0);
    float o = 0.0f;
    float d = A.sinks ? 1.0f : 0.0f;
    for (int t0 = 0; t0 < ctx; t0 += 32) {
        const int n = min(32, ctx - t0);
        float vb[32], eb[32];
#pragma unroll
        for (int j = 0; j < 32; j++) {
            int t = t0 + j < ctx ? t0 + j : ctx - 1;
            int slot = (s0 + t) % A.slot_count;
            vb[j] = vbase[(size_t)slot * A.value_stride];
            eb[j] = ef[(size_t)t * 4];
        }
        const uint32_t bits = mk[t0 >> 5];
        if (bits == 0 && n == 32) {
#pragma unroll
            for (int j = 0; j < 32; j++) {
                o = fmaf(eb[j], vb[j], o);
                d = d + eb[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 32; j++) {
                if (j < n) {
                    if ((bits >> j) & 1u) {
                        if (x4)
                            o = fmaf(vb[j], 1.0f, o * eb[j]);  // affine_add: fma(value, 1, out*old)
                        else
                            o = fmaf(o, eb[j], vb[j]);         // scale_add: fma(out, old, value)
                        float p = d * eb[j];
                        d = p + 1.0f;
                    } else {
                        o = fmaf(eb[j], vb[j], o);             // axpy / affine_add with mul 1
                        d = d + eb[j];
                    }
                }
            }
        }
    }
    if (dim_ok) A.out[(size_t)head * A.vd + dim] = o;
    if (slice == 0 && lane == 0) A.den[head] = d;
}

// D: out = out * (1/den) where den > 0 (the reference's final scale), and
// optionally the Q8_K quantization of the result for the next projection.
__global__ __launch_bounds__(256) void attn_exact_finish_kernel(float *out, const float *den, int vd, int n, XQ xq) {
    __shared__ float red[4];
    const int e = blockIdx.x * 256 + threadIdx.x;
    float v = 0.0f;
    if (e < n) {
        v = out[e];
        const float d = den[e / vd];
        if (d > 0.0f) {
            const float inv = 1.0f / d;
            v = v * inv;
        }
        out[e] = v;
    }
    if (xq.qs) q8k_block_store(v, blockIdx.x, e, xq, red);
}

}  // namespace rh
