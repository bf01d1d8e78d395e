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
//      Each step gets one coefficient: the weight w = expf(s - max) on an
//      ordinary step, the old-output multiplier old = expf(max - s) on a new
//      maximum (flagged in a bit mask).  The grouped form is then
//      o = fma(a, v, o*m) with (a, m) = (w, 1) or (1, old) (o*1 is exact).
//   C  attn_exact_chain:   the FMA recurrences, one lane per (head, dim),
//      V streamed into LDS by direct global->LDS loads; the denominators run
//      as the same recurrence with v = 1.
//   D  attn_exact_finish:  out = out * (1/denom), fused with the Q8_K
//      quantization the output projection needs.
// Which update form a head uses follows the reference: affine_add_f32x4
// (fma(v, alpha, out*mul)) for heads 0..3 of kv_mul 4/6 groups, scale_add /
// axpy (fma(out, old, v) / fma(w, v, out)) otherwise; with sinks every head
// uses the per-head sink scan (online_attention_with_sink).
#pragma once
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

// tab: the 2^(k/N) table (kExp2fTab, or a copy of it in LDS).  Branch-free:
// the main path runs for every input (its table index is always in range)
// and the special cases of glibc's |x| >= 88 branch are selected after it:
// -inf -> 0, NaN -> x + x, +inf and x > 0x1.62e42ep6 -> inf, x <
// -0x1.9fe368p6 -> 0; the rest of that range takes the main path there too.
__device__ __forceinline__ float expf_glibc_tab(float x, const uint64_t *tab) {
    const double invln2n = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32768.0, c1 = 0x1.ebfce50fac4f3p-3 / 1024.0,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    double xd = (double)x;
    double kd = __builtin_fma(invln2n, xd, shift);
    uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    double r = __builtin_fma(invln2n, xd, -kd);
    uint64_t t = tab[ki % 32] + (ki << 47);
    double s = __builtin_bit_cast(double, t);
    double z = __builtin_fma(c0, r, c1);
    double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    float res = (float)y;
    asm volatile("" : "+v"(res));  // the main path runs on every lane: no branch around it
    res = x > 0x1.62e42ep6f ? __builtin_bit_cast(float, 0x7f800000u) : res;
    res = x < -0x1.9fe368p6f ? 0.0f : res;
    return __builtin_isnan(x) ? x + x : res;
}
__device__ __forceinline__ float expf_glibc(float x) { return expf_glibc_tab(x, kExp2fTab); }

struct AttnExactArgs {
    const float *q;      // [n_heads * hd]
    const float *k;      // cache base, slot s, kv head h at k + s*key_stride + h*hd
    const float *v;
    const float *sinks;  // [n_heads] or null
    float *scores;       // [n_heads][cap]   q.k * scale per position
    float *e;            // [n_heads][cap]   expf(s - max), or on a new max expf(old max - s) (0 from -inf)
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
    // Several query tokens in one launch (prefill), token z = blockIdx.z at
    // position pos0 + z: its query at q + z*q_tok, its output at out +
    // z*o_tok, its own scratch block tok_scratch floats further per token.
    // n_tok = 0: one token, ranges from st or start_t/end_t.
    int32_t n_tok, pos0;
    int64_t q_tok, o_tok, tok_scratch;
    // Optional tiled transposed V copy (vt4_off layout, vt_stride slots per
    // column): with a range starting on a multiple of 4 positions and not
    // wrapping, the chain kernel streams V from it, a 16-dim slice's tile in
    // one contiguous 4 KB block, so that one 16-byte LDS read gives a lane
    // four steps of its value dim.  null: V only.
    const float *vt;
    int32_t vt_stride;
    // Decode only (n_tok = 0): the lane-sliced scores kernel also does the
    // RoPE + KV store of the current position (rope_kv_kernel's work) from
    // the raw q/k/v in rope, so that launch is not needed.
    RopeArgs rope;
    int32_t fuse_rope;
    // 1: the K and V caches hold bf16 (attention_over_kv_heads_bf16,
    // src/model.rs:6205-6580): rows widened on load, every head's scores in
    // dot_bf16_f32's single-accumulator order, V from the f32 tiled copy
    // (widened bf16 values) or, without it, widened from the rows
    int32_t kv_bf16;
    // Ring layers in a multi-token launch (lin = 1): k and v are a linear
    // buffer whose row r holds position lin_pos0 + r (the ring's positions
    // before the chunk, then the chunk's own), and every token reads the ring
    // as it stood at its own step: slot s (of slot_count) holds the latest
    // position <= the token's that is congruent to s.  tok_view sets lin_b
    // and lin_c for the token; kv_row maps a slot to its buffer row.
    int32_t lin, lin_pos0, lin_b, lin_c;
    // Streamed decode launch (attn_exact_stream_kernel): scores and chain
    // workgroups in one grid; sync = [epoch, ticket, timeouts, flags
    // [n_kv][cap/64]] (zeroed once when allocated), ep = the epoch the
    // launch reads at its start.  null: separate launches.
    uint32_t *sync;
    uint32_t ep;
    // Streamed launch only, optional: the next GEMV's weight rows (pf_rows
    // rows at pf_stride bytes), which its persistent grid (a multiple of 8
    // workgroups) takes in groups of pf_group_rows rows round robin over the
    // workgroups; the scores workgroups, once their tiles are scored, load
    // the groups their XCD will compute into that XCD's L2.  null: none.
    const uint8_t *pf;
    int64_t pf_stride;
    int32_t pf_rows, pf_group_rows;
};

// Element e of a head vector x after RoPE with the row's cos/sin, exactly as
// rope_kv_kernel computes it (interleaved pairs (2p, 2p+1) or NeoX pairs
// (p, p + hd/2); r0 = v0*c - v1*s, r1 = v0*s + v1*c).
__device__ __forceinline__ float rope_elem(const float *x, int e, int half, bool neox, const float *ct,
                                           const float *st) {
    int p, i0, i1;
    if (neox) {
        p = e < half ? e : e - half;
        i0 = p;
        i1 = p + half;
    } else {
        p = e >> 1;
        i0 = 2 * p;
        i1 = i0 + 1;
    }
    const float c = ct[p], s = st[p], v0 = x[i0], v1 = x[i1];
    return e == i0 ? v0 * c - v1 * s : v0 * s + v1 * c;
}

// The single-token view of token blockIdx.z of a multi-token launch: its
// range is start_t (or the window's start) ..= pos0 + z.
__device__ __forceinline__ AttnExactArgs tok_view(const AttnExactArgs &A0) {
    if (A0.n_tok == 0) return A0;
    AttnExactArgs A = A0;
    const int z = blockIdx.z;
    const int64_t sc = (int64_t)z * A0.tok_scratch;
    A.q += (int64_t)z * A0.q_tok;
    A.out += (int64_t)z * A0.o_tok;
    A.scores += sc;
    A.e += sc;
    A.tmax += sc;
    A.newmask += sc;
    A.den += sc;
    A.st = nullptr;
    A.end_t = A0.pos0 + z;
    A.start_t = A0.window > 0 ? max(0, A.end_t + 1 - A0.window) : A0.start_t;
    if (A0.lin) {
        A.lin_c = A.end_t % A0.slot_count;
        A.lin_b = A.end_t - A0.lin_pos0 - A.lin_c;
    }
    return A;
}

// The K/V row that holds ring slot `slot` (the slot itself unless lin).  A
// slot past the token's own position (read only by the scores kernels'
// speculative full-tile loads, whose rows are never used) has no row yet:
// it maps to row 0, so every load stays inside the buffer.
__device__ __forceinline__ int kv_row(const AttnExactArgs &A, int slot) {
    return A.lin ? max(0, slot + A.lin_b - (slot > A.lin_c ? A.slot_count : 0)) : slot;
}

// ---- streamed decode launch: flags between scores and chain workgroups -------
// A scores workgroup publishes tile `tile` of kv head h by storing epoch + 1
// in its flag after the scores (and the current position's K/V rows) are
// written back; chain workgroups wait for it before loading them, by loads
// coherent across the XCDs' L2 caches.  The scores workgroups never wait, and
// the chain workgroups take far fewer CUs than the device has, so every
// awaited flag is set within microseconds.  The wait is bounded all the same
// (about 20 ms): a wait that runs out marks the launch in sync[2] (epoch + 1)
// and every later wait of that launch returns at once, so a broken launch
// ends with wrong values, never a hang.
#define STREAM_SPIN_MAX (1 << 14)
__device__ __forceinline__ uint32_t *stream_flag(const AttnExactArgs &A, int h, int tile) {
    return A.sync + 3 + (size_t)h * (A.cap / 64) + tile;
}
// Waits until tiles 0..tile of kv head h are published; ready counts the
// tiles known to be (a prefix), and one poll reads the flags of the next 64
// tiles at once (one load per lane), so a run of published tiles costs one
// round trip, not one per tile.
__device__ __forceinline__ void stream_wait_prefix(const AttnExactArgs &A, int h, int tile, int ntiles, int &ready) {
    if (tile < ready) return;
    const int lane = threadIdx.x & 63;
    for (int it = 0; it < STREAM_SPIN_MAX; it++) {
        const int t = ready + lane;
        // the timeout mark and the flags in flight together (unconditional
        // loads, clamped index): one round trip per poll
        const uint32_t bad = __hip_atomic_load(A.sync + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t fv = __hip_atomic_load(stream_flag(A, h, min(t, ntiles - 1)), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t v = t < ntiles ? fv : A.ep + 1;
        const unsigned long long ok = __ballot(v == A.ep + 1);
        ready += ~ok == 0ull ? 64 : (int)__builtin_ctzll(~ok);  // the published run from `ready` on
        if (tile < ready) return;
        if (__builtin_amdgcn_readfirstlane(bad) == A.ep + 1) {
            ready = ntiles;
            return;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    __hip_atomic_store(A.sync + 2, A.ep + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ready = ntiles;
}
__device__ __forceinline__ void stream_wait(const AttnExactArgs &A, int h, int tile) {
    const uint32_t *f = stream_flag(A, h, tile);
    for (int it = 0; it < STREAM_SPIN_MAX; it++) {
        const uint32_t bad = __hip_atomic_load(A.sync + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t v = __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__builtin_amdgcn_readfirstlane(v) == A.ep + 1) return;
        if (__builtin_amdgcn_readfirstlane(bad) == A.ep + 1) return;
        __builtin_amdgcn_s_sleep(2);
    }
    __hip_atomic_store(A.sync + 2, A.ep + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A store the streamed launch's other workgroups may read: device scope
// (sc1, written through the non-coherent L2), so no L2 write-back is needed
// before the flag that publishes it.
__device__ __forceinline__ void st_pub(float *p, float v, bool coherent) {
    if (coherent) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}
// A 16-byte direct global->LDS load that bypasses the non-coherent L2 (sc1).
__device__ __forceinline__ void dma16_coherent(const void *src, void *lds) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t *)lds, 16, 0, 16);
}

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
#define CH_MAXG 8    // query heads per kv head handled by the lane-sliced scores and chain kernels

// e of (kv head h, head g of its group, position t).
__device__ __forceinline__ size_t e_index(const AttnExactArgs &A, int h, int g, int t) {
    return (size_t)(h * A.kv_mul + g) * A.cap + t;
}

// A: one workgroup per (tile of EX_TILE positions, kv head).  Writes the
// scores of every query head of the group and each head's tile maximum.
__global__ __launch_bounds__(256) void attn_exact_scores_kernel(AttnExactArgs A0) {
    const AttnExactArgs A = tok_view(A0);
    extern __shared__ float s_dyn[];
    const int hd = A.hd, kvm = A.kv_mul;
    // Row pitch hd + 8: the x4 path's 8-lane groups read 8 consecutive floats
    // of four rows per half-wave, which then fall in 32 distinct banks.
    const int ldk = hd + 8;
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
    const uint16_t *kh16 = (const uint16_t *)A.k + (size_t)h * hd;
    const int h4 = hd >> 2;
    if (A.kv_bf16) {
#pragma unroll 4
        for (int i = tid; i < nt * hd; i += 256) {
            int tt = i / hd, c = i - tt * hd;
            int slot = (s0 + t_base + tt) % A.slot_count;
            s_k[tt * ldk + c] = bf16_to_f32(kh16[(size_t)kv_row(A, slot) * A.key_stride + c]);
        }
    } else if (A.kvec && (256 % h4) == 0 && A.slot_count >= EX_TILE) {
        // thread -> (row r0 + k*rstep, float4 column c): one division, and the
        // ring wrap as a compare (a tile spans fewer rows than the ring)
        const int r0 = tid / h4, c = (tid - r0 * h4) * 4, rstep = 256 / h4;
        const int base = (s0 + t_base) % A.slot_count;
#pragma unroll 8
        for (int tt = r0; tt < nt; tt += rstep) {
            int slot = base + tt;
            if (slot >= A.slot_count) slot -= A.slot_count;
            *(float4 *)(s_k + tt * ldk + c) = *(const float4 *)(kh + (size_t)kv_row(A, slot) * A.key_stride + c);
        }
    } else {
#pragma unroll 4
        for (int i = tid; i < nt * hd; i += 256) {
            int tt = i / hd, c = i - tt * hd;
            int slot = (s0 + t_base + tt) % A.slot_count;
            s_k[tt * ldk + c] = kh[(size_t)kv_row(A, slot) * A.key_stride + c];
        }
    }
    __syncthreads();
    // x4 heads: 8 lanes per (head, position), one accumulator per lane,
    // chained over the hd/8 chunks, then hsum_avx.
    const int nx4 = A.kv_bf16 ? kvm : ((A.sinks == nullptr && (kvm == 4 || kvm == 6)) ? 4 : 0);
    // (head g, row tt) pairs are numbered g*EX_TILE + tt, rows past nt idle
    {
        const int pairs = nx4 * EX_TILE;
        const int l = lane & 7;
        for (int p0 = wave * 8; p0 < pairs; p0 += 32) {
            const int p = p0 + (lane >> 3);
            const int g = p / EX_TILE, tt = p % EX_TILE;
            const bool ok = tt < nt;
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
    // other heads: dot_f32_avx2 (src/simd.rs:6547-6586): four 8-wide
    // accumulators over 32-element chunks, (a0+a1)+(a2+a3), the 8-chunk tail,
    // hsum_avx, then the scalar tail.  8 lanes per (head, position), lane l
    // holding vector lane l of all four accumulators.
    {
        const int ng = kvm - nx4;
        const int pairs = ng * EX_TILE;
        const int l = lane & 7;
        const int main32 = hd / 32, tail8 = (hd - main32 * 32) / 8;
        for (int p0 = wave * 8; p0 < pairs; p0 += 32) {
            const int p = p0 + (lane >> 3);
            const int tt = p % EX_TILE;
            const bool ok = tt < nt;
            const int g = nx4 + p / EX_TILE;
            const float *qq = s_q + g * hd, *kk = s_k + tt * ldk;
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
            if (ok)
                for (int c = 0; c < main32; c++) {
                    a0 = fmaf(qq[32 * c + l], kk[32 * c + l], a0);
                    a1 = fmaf(qq[32 * c + 8 + l], kk[32 * c + 8 + l], a1);
                    a2 = fmaf(qq[32 * c + 16 + l], kk[32 * c + 16 + l], a2);
                    a3 = fmaf(qq[32 * c + 24 + l], kk[32 * c + 24 + l], a3);
                }
            float y = (a0 + a1) + (a2 + a3);
            if (ok)
                for (int i = 0; i < tail8; i++) y = fmaf(qq[32 * main32 + 8 * i + l], kk[32 * main32 + 8 * i + l], y);
            float a = y + __shfl_xor(y, 4, 64);
            float b = a + __shfl_xor(a, 1, 64);
            float d = b + __shfl_xor(b, 2, 64);
            if (ok && l == 0) {
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

// A, head dims that are multiples of 32 up to 128: the K tile is staged in
// LDS per row as [AVX2 lane l][m] (element 8m + l), so lane l of an 8-lane
// group reads its hd/8 elements with hd/32 16-byte reads; q's slice for the
// same lane sits in registers.  One wave per query head (64 positions x 8
// lanes), the per-lane accumulation in the reference's order:
//   dot_f32x4_avx2 (heads 0..3 of kv_mul 4/6): acc = fma(q, k, acc) over m;
//   dot_f32_avx2 (the others): four accumulators over m = 4c + j, then
//   (a0 + a1) + (a2 + a3);
// then hsum_avx across the 8 lanes.  Writes the same scores and tile maxima
// as attn_exact_scores_kernel.
// v of lane i + N of this lane's 16-lane row (lanes whose source lies past
// the row end are not used by the callers).
template <int N>
__device__ __forceinline__ float row_shl(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x100 + N, 0xF, 0xF, false));
}

// Tile `tile` of kv head h by threads 0-255 of the workgroup; returns false
// when the tile lies past the range (nothing written).
template <int HD>
__device__ __forceinline__ bool scores8_tile(const AttnExactArgs &A, int tile, int h) {
    constexpr int M = HD / 8;        // elements per lane
    constexpr int LS = M + 4;        // LDS floats per lane slice (padded: a row's 8 slices hit distinct banks)
    constexpr int RS = 8 * LS;       // LDS floats per K row
    __shared__ __align__(16) float s_k[EX_TILE * RS];
    __shared__ __align__(16) float s_q[CH_MAXG * RS];  // the heads' q, lane-sliced like a K row
    __shared__ float s_sc[CH_MAXG * EX_TILE];
    const int t_base = tile * EX_TILE;
    const int tid = threadIdx.x, lane = tid & 63, kvm = A.kv_mul;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const float *kh = A.k + (size_t)h * HD;
    const uint16_t *kh16 = (const uint16_t *)A.k + (size_t)h * HD;
    // the K tile's loads first (registers), so their latency overlaps the q
    // staging below; element 4*c4 + i of a row goes to lane slice
    // (4*c4 + i) % 8, position (4*c4 + i) / 8
    constexpr int H4 = HD / 4, RSTEP = 256 / H4, NKR = EX_TILE / RSTEP;
    const int r0 = tid / H4, c4 = tid - r0 * H4;
    float4 kreg[NKR];
    auto load_k = [&](int start, int rows) {
        const int base = (start + t_base) % A.slot_count;
#pragma unroll
        for (int i = 0; i < NKR; i++) {
            int slot = base + min(r0 + i * RSTEP, rows - 1);
            if (slot >= A.slot_count) slot -= A.slot_count;
            const size_t kr = (size_t)kv_row(A, slot) * A.key_stride + 4 * c4;
            kreg[i] = A.kv_bf16 ? bf16x4_load(kh16 + kr) : *(const float4 *)(kh + kr);
        }
    };
    // Without a window the range starts at start_t, which the host passes as
    // a hint (A.start_t) when the range comes from the device state: the
    // tile's K loads are issued before that state arrives, every row of the
    // tile (slots wrap, so any start is in bounds; rows past the range are
    // never used), and issued again below if the range starts elsewhere.
    const bool spec = A.window == 0;
    if (spec) load_k(A.start_t, EX_TILE);
    // q of the kv head's query heads, both elements of each RoPE pair, loaded
    // before the range (the device step state) arrives: only the cos/sin row
    // waits for the position
    const RopeArgs &RA = A.rope;
    const int half = HD / 2;
    constexpr int QI = (CH_MAXG * HD + 255) / 256;  // elements per thread
    const float *qsrc = (A.fuse_rope ? RA.q : A.q) + (size_t)h * kvm * HD;
    float qv0[QI], qv1[QI];
#pragma unroll
    for (int u = 0; u < QI; u++) {
        const int i = min(tid + 256 * u, kvm * HD - 1);
        const int g = i / HD, e = i - g * HD;
        const int p = RA.neox ? (e < half ? e : e - half) : e >> 1;
        const int i0 = RA.neox ? p : 2 * p, i1 = RA.neox ? p + half : 2 * p + 1;
        qv0[u] = qsrc[g * HD + i0];
        qv1[u] = qsrc[g * HD + i1];
    }
    int s0, e0;
    exact_range(A, s0, e0);
    const int ctx = e0 - s0 + 1;
    if (ctx <= 0 || t_base >= ctx) return false;
    const int nt = min(EX_TILE, ctx - t_base);
    if (!spec || s0 != A.start_t) load_k(s0, nt);
    // fused RoPE: the current position e0 and its cos/sin row
    const bool fuse = A.fuse_rope != 0 && e0 < RA.max_pos;
    const float *ct = RA.cos_t + (size_t)e0 * half, *stb = RA.sin_t + (size_t)e0 * half;
    {
        // (rotated here when RoPE is fused, as rope_elem / rope_kv_kernel:
        // r0 = v0*c - v1*s, r1 = v0*s + v1*c), element e of head g at lane
        // slice e % 8, position e / 8
#pragma unroll
        for (int u = 0; u < QI; u++) {
            const int i = tid + 256 * u;
            if (i < kvm * HD) {
                const int g = i / HD, e = i - g * HD;
                const int p = RA.neox ? (e < half ? e : e - half) : e >> 1;
                const bool first = RA.neox ? e < half : (e & 1) == 0;
                float v = first ? qv0[u] : qv1[u];
                if (fuse) {
                    const float c = ct[p], sn = stb[p];
                    v = first ? qv0[u] * c - qv1[u] * sn : qv0[u] * sn + qv1[u] * c;
                }
                s_q[g * RS + (e & 7) * LS + (e >> 3)] = v;
            }
        }
    }
    {
        const int lbase = (4 * c4) & 7, m = (4 * c4) >> 3;
#pragma unroll
        for (int i = 0; i < NKR; i++) {
            float *d = s_k + (r0 + i * RSTEP) * RS + m;
            d[(lbase + 0) * LS] = kreg[i].x;
            d[(lbase + 1) * LS] = kreg[i].y;
            d[(lbase + 2) * LS] = kreg[i].z;
            d[(lbase + 3) * LS] = kreg[i].w;
        }
    }
    const int l = lane & 7, sub = lane >> 3;
    const int tt_cur = e0 - s0 - t_base;  // the current position's row, if in this tile
    if (fuse && tt_cur >= 0 && tt_cur < EX_TILE) {
        // k rotated into the tile (over the cache row staged above) and both
        // cache rows of the current position stored, as rope_kv_kernel does
        __syncthreads();
        const int slot = RA.ring ? e0 % RA.slots : e0 - RA.slot_off;
        const int kvd = RA.n_kv * HD, vvd = RA.n_kv * RA.vd;
        for (int e = tid; e < HD; e += 256) {
            float kr = rope_elem(RA.k + (size_t)h * HD, e, half, RA.neox != 0, ct, stb);
            if (RA.kv_bf16) {
                const uint16_t kb = f32_to_bf16(kr);
                ((uint16_t *)RA.kcache)[(size_t)slot * kvd + h * HD + e] = kb;
                kr = bf16_to_f32(kb);  // the score reads the stored (bf16) key
            } else {
                st_pub(RA.kcache + (size_t)slot * kvd + h * HD + e, kr, A.sync != nullptr);
            }
            s_k[tt_cur * RS + (e & 7) * LS + (e >> 3)] = kr;
        }
        for (int e = tid; e < RA.vd; e += 256) {
            float v = RA.v[(size_t)h * RA.vd + e];
            if (RA.kv_bf16) {
                const uint16_t vb = f32_to_bf16(v);
                ((uint16_t *)RA.vcache)[(size_t)slot * vvd + h * RA.vd + e] = vb;
                v = bf16_to_f32(vb);
            } else {
                st_pub(RA.vcache + (size_t)slot * vvd + h * RA.vd + e, v, A.sync != nullptr);
            }
            if (RA.vtcache) st_pub(RA.vtcache + vt4_off(h * RA.vd + e, slot, RA.vt_stride), v, A.sync != nullptr);
        }
    }
    __syncthreads();
    for (int g = wave; g < kvm; g += 4) {
        // dot_f32x4 / dot_bf16x4 / dot_bf16_f32: one accumulator per lane;
        // dot_f32_avx2: four
        const bool x4 = A.kv_bf16 || (A.sinks == nullptr && (kvm == 4 || kvm == 6) && g < 4);
        float q[M];
        {
            const float *qr = s_q + g * RS + l * LS;
#pragma unroll
            for (int r = 0; r < M / 4; r++) {
                const float4 f = *(const float4 *)(qr + 4 * r);
                q[4 * r] = f.x;
                q[4 * r + 1] = f.y;
                q[4 * r + 2] = f.z;
                q[4 * r + 3] = f.w;
            }
        }
        // two positions per step (tt and tt + 32), so two independent
        // accumulation chains interleave; the form is chosen once per head
        auto run = [&](auto x4c) {
            constexpr bool X4 = decltype(x4c)::value;
#pragma unroll
            for (int it = 0; it < EX_TILE / 16; it++) {
                float y[2];
                float k[2][M];
#pragma unroll
                for (int p = 0; p < 2; p++) {
                    const float *kr = s_k + (8 * it + 32 * p + sub) * RS + l * LS;
#pragma unroll
                    for (int r = 0; r < M / 4; r++) {
                        const float4 f = *(const float4 *)(kr + 4 * r);
                        k[p][4 * r] = f.x;
                        k[p][4 * r + 1] = f.y;
                        k[p][4 * r + 2] = f.z;
                        k[p][4 * r + 3] = f.w;
                    }
                }
                if (X4) {
                    y[0] = 0.0f;
                    y[1] = 0.0f;
#pragma unroll
                    for (int mm = 0; mm < M; mm++) {
                        y[0] = fmaf(q[mm], k[0][mm], y[0]);
                        y[1] = fmaf(q[mm], k[1][mm], y[1]);
                    }
                } else {
#pragma unroll
                    for (int p = 0; p < 2; p++) {
                        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int c = 0; c < M / 4; c++)
#pragma unroll
                            for (int j = 0; j < 4; j++) a[j] = fmaf(q[4 * c + j], k[p][4 * c + j], a[j]);
                        y[p] = (a[0] + a[1]) + (a[2] + a[3]);
                    }
                }
#pragma unroll
                for (int p = 0; p < 2; p++) {
                    // hsum_avx of the 8 lanes, needed in lane l = 0 only: lane i
                    // takes lane i + N of its row (DPP row_shl), so lanes 0 and 8
                    // of every row get (y0 + y4) + (y1 + y5) and (y2 + y6) +
                    // (y3 + y7) and their sum, as the xor-4/1/2 butterfly gives
                    const float a = y[p] + row_shl<4>(y[p]);
                    const float b = a + row_shl<1>(a);
                    const float d = b + row_shl<2>(b);
                    if (l == 0) s_sc[g * EX_TILE + 8 * it + 32 * p + sub] = d * A.scale;
                }
            }
        };
        if (x4) run(std::true_type{});
        else run(std::false_type{});
    }
    __syncthreads();
    // coalesced score rows + tile maxima (max is exact in any order)
    const int ntl = A.cap / EX_TILE;
    for (int g = wave; g < kvm; g += 4) {
        const int head = h * kvm + g;
        float v = lane < nt ? s_sc[g * EX_TILE + lane] : -INFINITY;
        if (lane < nt) st_pub(A.scores + (size_t)head * A.cap + t_base + lane, v, A.sync != nullptr);
        const float mx = wave_max(v);
        if (lane == 0) A.tmax[(size_t)head * ntl + tile] = mx;
    }
    return true;
}
template <int HD>
__global__ __launch_bounds__(256) void attn_exact_scores8_kernel(AttnExactArgs A0) {
    const AttnExactArgs A = tok_view(A0);
    scores8_tile<HD>(A, blockIdx.x, blockIdx.y);
}

// A for many query tokens at once (prefill without a window or ring view:
// every token's range starts at start_t, so all tokens share the tile
// boundaries).  One workgroup per (tile, kv head, block of MQ_PAIRS / kv_mul
// consecutive tokens): the K tile is staged once, lane-sliced as in
// scores8_tile, and each wave holds 16 of its positions in registers
// (positions 16w + 8p + sub, p = 0, 1) while it walks the block's
// (token, head) pairs, whose q slices are read from LDS.  Per pair and
// position the lane arithmetic is scores8_tile's (dot_f32x4 / dot_bf16 one
// accumulator, dot_f32_avx2 four, then the row_shl hsum and the scale), so
// every token's scores and tile maxima equal its single-token launch's.
// Tokens whose range ends before the tile write nothing.
#define MQ_PAIRS 32
__host__ __device__ inline int mq_tokens(int kvm) { return kvm >= MQ_PAIRS ? 1 : MQ_PAIRS / kvm; }
template <int HD>
__global__ __launch_bounds__(256) void attn_exact_scores_mq_kernel(AttnExactArgs A) {
    // q slices padded (LS: a pair's eight slices in distinct banks, read once
    // per pair); K slices unpadded (LSK, read once per wave), and the staged
    // scores over the K tile once every wave holds its K in registers: 52 KB
    // at HD 128, three workgroups per CU
    constexpr int M = HD / 8, LS = M + 4, RS = 8 * LS, LSK = M, RSK = 8 * LSK;
    static_assert(MQ_PAIRS * EX_TILE <= EX_TILE * RSK, "the score staging fits in the K tile");
    __shared__ __align__(16) float s_k[EX_TILE * RSK];
    __shared__ __align__(16) float s_q[MQ_PAIRS * RS];
    float *s_sc = s_k;
    const int kvm = A.kv_mul, qb = mq_tokens(kvm);
    const int tile = blockIdx.x, h = blockIdx.y, z0 = blockIdx.z * qb;
    const int nz = min(qb, A.n_tok - z0), npair = nz * kvm;
    const int t_base = tile * EX_TILE;
    // the block's last token has the longest range
    const int ctx_last = A.pos0 + z0 + nz - 1 - A.start_t + 1;
    if (nz <= 0 || ctx_last <= t_base) return;
    const int rows = min(EX_TILE, ctx_last - t_base);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    {
        // K rows t_base.. (clamped to the rows any token of the block reads)
        constexpr int H4 = HD / 4, RSTEP = 256 / H4, NKR = EX_TILE / RSTEP;
        const int r0 = tid / H4, c4 = tid - r0 * H4;
        const float *kh = A.k + (size_t)h * HD;
        const uint16_t *kh16 = (const uint16_t *)A.k + (size_t)h * HD;
        // every load (the K tile's rows, then the pairs' q rows: float4
        // column c of pair pr, clamped to the last pair) issued before any
        // LDS store, in straight-line code
        float4 kreg[NKR];
        size_t kr[NKR];
#pragma unroll
        for (int i = 0; i < NKR; i++)
            kr[i] = (size_t)((A.start_t + t_base + min(r0 + i * RSTEP, rows - 1)) % A.slot_count) * A.key_stride +
                    4 * c4;
        if (A.kv_bf16) {
#pragma unroll
            for (int i = 0; i < NKR; i++) kreg[i] = bf16x4_load(kh16 + kr[i]);
        } else {
#pragma unroll
            for (int i = 0; i < NKR; i++) kreg[i] = *(const float4 *)(kh + kr[i]);
        }
        constexpr int NQ4 = MQ_PAIRS * H4 / 256;
        float4 qreg[NQ4];
#pragma unroll
        for (int u = 0; u < NQ4; u++) {
            const int idx = tid + 256 * u, pr = min(idx / H4, npair - 1), c = idx - (idx / H4) * H4;
            const int zz = pr / kvm, g = pr - zz * kvm;
            qreg[u] = *(const float4 *)(A.q + (int64_t)(z0 + zz) * A.q_tok + (size_t)(h * kvm + g) * HD + 4 * c);
        }
        // q of every (token, head) pair, lane-sliced like a K row
#pragma unroll
        for (int u = 0; u < NQ4; u++) {
            const int idx = tid + 256 * u, pr = idx / H4, e = 4 * (idx - pr * H4);
            if (pr < npair) {
                float *d = s_q + pr * RS + (e >> 3);
                d[((e + 0) & 7) * LS] = qreg[u].x;
                d[((e + 1) & 7) * LS] = qreg[u].y;
                d[((e + 2) & 7) * LS] = qreg[u].z;
                d[((e + 3) & 7) * LS] = qreg[u].w;
            }
        }
        const int lbase = (4 * c4) & 7, m = (4 * c4) >> 3;
#pragma unroll
        for (int i = 0; i < NKR; i++) {
            float *d = s_k + (r0 + i * RSTEP) * RSK + m;
            d[(lbase + 0) * LSK] = kreg[i].x;
            d[(lbase + 1) * LSK] = kreg[i].y;
            d[(lbase + 2) * LSK] = kreg[i].z;
            d[(lbase + 3) * LSK] = kreg[i].w;
        }
    }
    __syncthreads();
    const int l = lane & 7, sub = lane >> 3;
    float k[2][M];
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const float *kr = s_k + (16 * wave + 8 * p + sub) * RSK + l * LSK;
#pragma unroll
        for (int r = 0; r < M / 4; r++) {
            const float4 f = *(const float4 *)(kr + 4 * r);
            k[p][4 * r] = f.x;
            k[p][4 * r + 1] = f.y;
            k[p][4 * r + 2] = f.z;
            k[p][4 * r + 3] = f.w;
        }
    }
    __syncthreads();  // every wave holds its K: the tile's LDS now takes the scores
    // pair pr's q slice; pairs two at a time, so four independent chains
    // (two pairs x two positions) interleave, and both pairs' reads go out
    // together
    auto read_q = [&](int pr, float (&q)[M]) {
        const float *qr = s_q + pr * RS + l * LS;
#pragma unroll
        for (int r = 0; r < M / 4; r++) {
            const float4 f = *(const float4 *)(qr + 4 * r);
            q[4 * r] = f.x;
            q[4 * r + 1] = f.y;
            q[4 * r + 2] = f.z;
            q[4 * r + 3] = f.w;
        }
    };
    // one pair's two positions in scores8_tile's lane arithmetic (x4: one
    // accumulator; dot_f32_avx2: four, then (a0 + a1) + (a2 + a3))
    auto dots = [&](bool x4, const float (&q)[M], float (&y)[2]) {
        if (x4) {
            y[0] = 0.0f;
            y[1] = 0.0f;
#pragma unroll
            for (int mm = 0; mm < M; mm++) {
                y[0] = fmaf(q[mm], k[0][mm], y[0]);
                y[1] = fmaf(q[mm], k[1][mm], y[1]);
            }
        } else {
#pragma unroll
            for (int p = 0; p < 2; p++) {
                float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int c = 0; c < M / 4; c++)
#pragma unroll
                    for (int j = 0; j < 4; j++) a[j] = fmaf(q[4 * c + j], k[p][4 * c + j], a[j]);
                y[p] = (a[0] + a[1]) + (a[2] + a[3]);
            }
        }
    };
    auto store = [&](int pr, const float (&y)[2]) {
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const float a = y[p] + row_shl<4>(y[p]);
            const float b = a + row_shl<1>(a);
            const float d = b + row_shl<2>(b);
            if (l == 0) s_sc[pr * EX_TILE + 16 * wave + 8 * p + sub] = d * A.scale;
        }
    };
    // the x4 form: every head of a bf16 cache, heads 0..3 of a kv_mul 4/6
    // group without sinks (as scores8_tile)
    const bool bf = A.kv_bf16 != 0, gx = A.sinks == nullptr && (kvm == 4 || kvm == 6);
    int g = 0;  // head of pair pr within its group
    for (int pr = 0; pr < npair; pr += 2) {
        const int pr1 = min(pr + 1, npair - 1), g1 = g + 1 == kvm ? 0 : g + 1;
        float qa[M], qb[M], ya[2], yb[2];
        read_q(pr, qa);
        read_q(pr1, qb);
        const bool xa = bf || (gx && g < 4), xb = bf || (gx && g1 < 4);
        if (xa == xb) {
            // the same form: the two pairs' chains interleaved
            if (xa) {
                ya[0] = ya[1] = yb[0] = yb[1] = 0.0f;
#pragma unroll
                for (int mm = 0; mm < M; mm++) {
                    ya[0] = fmaf(qa[mm], k[0][mm], ya[0]);
                    ya[1] = fmaf(qa[mm], k[1][mm], ya[1]);
                    yb[0] = fmaf(qb[mm], k[0][mm], yb[0]);
                    yb[1] = fmaf(qb[mm], k[1][mm], yb[1]);
                }
            } else {
                dots(false, qa, ya);
                dots(false, qb, yb);
            }
        } else {
            dots(xa, qa, ya);
            dots(xb, qb, yb);
        }
        store(pr, ya);
        if (pr + 1 < npair) store(pr + 1, yb);
        g = g1 + 1 == kvm ? 0 : g1 + 1;
    }
    __syncthreads();
    // coalesced score rows and tile maxima of the tokens whose range reaches
    // the tile, each into its own scratch block
    const int ntl = A.cap / EX_TILE;
    for (int pr = wave; pr < npair; pr += 4) {
        const int zz = pr / kvm, g = pr - zz * kvm, z = z0 + zz;
        const int ctx = A.pos0 + z - A.start_t + 1;
        if (ctx <= t_base) continue;
        const int nt = min(EX_TILE, ctx - t_base);
        const int head = h * kvm + g;
        const int64_t sc = (int64_t)z * A.tok_scratch;
        const float v = lane < nt ? s_sc[pr * EX_TILE + lane] : -INFINITY;
        if (lane < nt) A.scores[sc + (size_t)head * A.cap + t_base + lane] = v;
        const float mx = wave_max(v);
        if (lane == 0) A.tmax[sc + (size_t)head * ntl + tile] = mx;
    }
}

// B: one wave per (tile of 64 positions, query head), four tiles per workgroup.  The running max before
// each step is max(initial, maxima of the earlier tiles, prefix max inside the
// tile), so every step's branch and expf argument are known without a serial
// scan.  On a new max the step's coefficient is isfinite(run) ? expf(run -
// s) : 0 (the factor the old output and denominator are scaled by; its own
// weight is 1), otherwise expf(s - run); the new-max steps are marked in
// newmask.
__global__ __launch_bounds__(256) void attn_exact_coef_kernel(AttnExactArgs A0) {
    const AttnExactArgs A = tok_view(A0);
    int s0, e0;
    exact_range(A, s0, e0);
    const int ctx = e0 - s0 + 1;
    // four tiles per workgroup, one per wave
    const int lane = threadIdx.x & 63, head = blockIdx.y;
    const int tile = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (ctx <= 0 || tile * EX_TILE >= ctx) return;
    const int ntl = A.cap / EX_TILE;
    const float *tm = A.tmax + (size_t)head * ntl;
    // both loads in flight together: this tile's scores and the maxima of
    // the tiles before it
    const int t = tile * EX_TILE + lane;
    const bool valid = t < ctx;
    const float s = A.scores[(size_t)head * A.cap + min(t, ctx - 1)];
    float m = -INFINITY;
    for (int j = lane; j < tile; j += 64) m = fmaxf(m, tm[j]);
    m = wave_max(m);
    if (A.sinks) m = fmaxf(A.sinks[head], m);
    // inclusive prefix max over lanes (DPP scan: within rows, then row 0-1
    // and 0-2 totals carried up; max is exact in any order), then each
    // lane's exclusive prefix from lane - 1 (wave_shr:1)
    float p = valid ? s : -INFINITY;
    p = dpp_max<0x111, 0xF>(p);
    p = dpp_max<0x112, 0xF>(p);
    p = dpp_max<0x114, 0xF>(p);
    p = dpp_max<0x118, 0xF>(p);
    p = dpp_max<0x142, 0xA>(p);
    p = dpp_max<0x143, 0xC>(p);
    const float prev = __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, p), __builtin_bit_cast(int, p), 0x138, 0xF, 0xF, false));
    const float run = lane == 0 ? m : fmaxf(m, prev);
    const bool flag = valid && s > run;
    float e = 0.0f;
    if (flag) {
        e = __builtin_isfinite(run) ? expf_glibc(run - s) : 0.0f;
    } else if (valid) {
        e = expf_glibc(s - run);
    }
    const int kvm = A.kv_mul, g = head % kvm;
    A.e[e_index(A, head / kvm, g, t)] = e;
    const unsigned long long bits = __ballot(flag);
    if (lane < 2) A.newmask[(size_t)head * (A.cap / 32) + 2 * tile + lane] = (uint32_t)(bits >> (32 * lane));
}

// C: the output and denominator recurrences
//   new max: out = affine_add: fma(v, 1, out*e) | scale_add: fma(out, e, v)
//            den = den*e + 1 (two roundings)
//   else:    out = fma(e, v, out);  den = den + e
// in the reference's step order.  A wave's own instruction stream is the
// limit here (one dependent FMA per step and lane, ~3 ns per instruction for
// a wave alone on its SIMD), so the recurrence waves issue nothing else but
// their LDS reads: e enters each FMA through its DPP row_newbcast operand
// (lane j of a 16-lane row holds step j), V comes from LDS, and producer
// waves stream both into a ring by direct global->LDS loads.

// Workgroup barrier without the memory-model waits of __syncthreads (which
// would drain the producers' loads); the asm statements keep the compiler
// from moving memory operations across it.
__device__ __forceinline__ void tile_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// e of step J broadcast from lane J of each row.
template <int J>
__device__ __forceinline__ float bcast16(float e16) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, e16), 0x150 + J, 0xF, 0xF, false));
}
__device__ __forceinline__ void bcast16_all(float e16, float *e) {
    e[0] = bcast16<0>(e16);   e[1] = bcast16<1>(e16);   e[2] = bcast16<2>(e16);   e[3] = bcast16<3>(e16);
    e[4] = bcast16<4>(e16);   e[5] = bcast16<5>(e16);   e[6] = bcast16<6>(e16);   e[7] = bcast16<7>(e16);
    e[8] = bcast16<8>(e16);   e[9] = bcast16<9>(e16);   e[10] = bcast16<10>(e16); e[11] = bcast16<11>(e16);
    e[12] = bcast16<12>(e16); e[13] = bcast16<13>(e16); e[14] = bcast16<14>(e16); e[15] = bcast16<15>(e16);
}

// 16 plain steps o = fma(e_j, v_j, o) with e_j taken straight from lane j of
// the row by the FMA's DPP operand (row_newbcast), so e costs no instruction
// of its own.  s_nop 1 gives the two wait states a DPP source needs after a
// VALU write.
__device__ __forceinline__ void cons_fma16_dpp(float e16, const float *v, float &o) {
    asm("s_nop 1\n\t"
        "v_fmac_f32_dpp %0, %1, %2 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %3 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %4 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %5 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %6 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %7 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %8 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %9 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %10 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %11 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %12 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %13 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %14 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %15 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %16 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %17 row_newbcast:15 row_mask:0xf bank_mask:0xf"
        : "+v"(o)
        : "v"(e16), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7]),
          "v"(v[8]), "v"(v[9]), "v"(v[10]), "v"(v[11]), "v"(v[12]), "v"(v[13]), "v"(v[14]), "v"(v[15]));
}

// 16 steps of the grouped update form on every step, o = fma(a_j, v_j, o*m_j)
// (the reference's affine_add_f32x4 with its new-max and ordinary cases, and
// the denominators with v = 1): a_j and m_j come from lane j of the row via
// row_newbcast, so a group holding new maxima runs branch-free in two DPP
// instructions per step.
__device__ __forceinline__ void cons_affine16_dpp(float a16, float m16, const float *v, float &o) {
#define RH_AFF(J, VJ)                                                               \
    "v_mul_f32_dpp %0, %2, %0 row_newbcast:" #J " row_mask:0xf bank_mask:0xf\n\t" \
    "v_fmac_f32_dpp %0, %1, %" #VJ " row_newbcast:" #J " row_mask:0xf bank_mask:0xf\n\t"
    asm("s_nop 1\n\t"
        RH_AFF(0, 3) RH_AFF(1, 4) RH_AFF(2, 5) RH_AFF(3, 6) RH_AFF(4, 7) RH_AFF(5, 8) RH_AFF(6, 9) RH_AFF(7, 10)
        RH_AFF(8, 11) RH_AFF(9, 12) RH_AFF(10, 13) RH_AFF(11, 14) RH_AFF(12, 15) RH_AFF(13, 16) RH_AFF(14, 17)
        RH_AFF(15, 18)
        : "+v"(o)
        : "v"(a16), "v"(m16), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7]),
          "v"(v[8]), "v"(v[9]), "v"(v[10]), "v"(v[11]), "v"(v[12]), "v"(v[13]), "v"(v[14]), "v"(v[15]));
#undef RH_AFF
}

// 16 recurrence steps with per-step new-max flags `bits`: the update forms
// selected per step (rare: only chunks holding a new maximum come here).
// e[j] is the weight of an ordinary step and the old-output factor of a
// flagged one.
template <bool DEN, bool X4>
__device__ __forceinline__ void chain_steps16_flags(const float *e, const float *v, float &o, uint32_t bits) {
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const float vj = DEN ? 1.0f : v[j];
        const float on = fmaf(e[j], vj, o);
        const float ox = (DEN || X4) ? fmaf(vj, 1.0f, o * e[j]) : fmaf(o, e[j], vj);
        o = ((bits >> j) & 1u) ? ox : on;
    }
}

// The grouped form's per-step pair for lane j of a 16-lane row from the
// step's coefficient and new-max bit (bit j of bits16): (a, m) = (e, 1) on
// an ordinary step, (1, e) on a new maximum.
__device__ __forceinline__ void aff_pair16(float e16, uint32_t bits16, int lane, float &a16, float &m16) {
    const bool nm = ((bits16 >> (lane & 15)) & 1u) != 0u;
    a16 = nm ? 1.0f : e16;
    m16 = nm ? e16 : 1.0f;
}

// C, four query heads per wave: chain workgroups, one per (kv head, group of
// four query heads, 16 value dims).  The consumer wave's four 16-lane rows
// are the four heads and lane % 16 the value dim, so all four rows read the
// same V element (one LDS broadcast) and each row takes its own head's
// coefficient through row_newbcast.  V of a kv head is then streamed from HBM
// once per layer, 64 B per position per workgroup.  A wave's direct loads
// complete at a fixed rate however many are in flight (about 75 ns per 64-lane
// 16-byte load of contiguous memory, about 130 ns when it touches sixteen
// separate 64-byte pieces), so the tile's loads are spread over five producer
// waves: four each load a quarter of the tile's V (16 positions x 16 dims, one
// contiguous KB of the tiled transposed copy), the fifth the four heads'
// scores.  Four coefficient waves, one per row, turn the scores into the
// steps' coefficients and new-max words in the ring (the coefficient stage,
// B, done here one group ahead of the recurrence instead of in a launch of
// its own).  The ring keeps C4_P tiles in flight; every wave meets at one
// barrier per C4_PER tiles.  The denominators run in a second kind of
// workgroup as the same DPP chain with v = 1.
#define C4_NT 16
#ifndef C4_P
#define C4_P 12
#endif
#ifndef C4_PER
#define C4_PER 4
#endif

struct Chain4Lds {
    float v[C4_NT][EX_TILE * 16];  // [slot][position][16 dims] (tiled copy: [position/4][16 dims][4])
    float e[C4_NT][4 * EX_TILE];   // [slot][row (head g0 + row)][position] coefficients
    uint32_t m[C4_NT][8];          // [slot][2 * row + word] new-max words
    float s[C4_NT][4 * EX_TILE];   // [slot][row][position] scores, for the coefficient waves
    uint64_t exp2tab[32];          // kExp2fTab for the coefficient waves' expf
};

template <int IPT>
__device__ __forceinline__ void c4_wait_tiles_after(int n_after) {
    switch (n_after) {
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
static_assert(C4_P - C4_PER <= 9, "c4_wait_tiles_after covers at most 9 tiles");
static_assert(2 * 9 <= 63, "vmcnt is 6 bits (up to two loads per producer per tile)");
static_assert(C4_NT >= C4_P + C4_PER, "ring too small");

// Producer protocol on the C4 ring: C4_P tiles are issued up front and every
// wave of the workgroup meets at a first barrier, then at one barrier per
// group.  Before group j's barrier the producer waits until the tiles of
// group j + LEAD have landed; after it, it issues the next C4_PER tiles,
// whose slots were last read in an earlier group.  LEAD = 0 feeds the
// recurrence wave (it reads group j after barrier j); LEAD = 1 feeds the
// coefficient waves, which work one group ahead (group j + 1 between barriers
// j and j + 1, group 0 between the first barrier and barrier 0).  issue(i)
// loads tile i into slot i % C4_NT.
template <int IPT, int LEAD, class Issue>
__device__ __forceinline__ void c4_producer_loop(int ntiles, Issue &issue) {
    const int ngroups = (ntiles + C4_PER - 1) / C4_PER;
    if (LEAD) {
        // the coefficient waves need only group 0 before the first barrier:
        // its tiles are issued and awaited first, the rest of the initial
        // window after that barrier (a streamed launch's issue waits for each
        // tile's flag, so the first barrier no longer waits for C4_P flags)
        for (int i = 0; i < min(C4_PER, ntiles); i++) issue(i);
        c4_wait_tiles_after<IPT>(0);
        tile_barrier();
        for (int i = C4_PER; i < min(C4_P, ntiles); i++) issue(i);
    } else {
        for (int i = 0; i < min(C4_P, ntiles); i++) issue(i);
        tile_barrier();
    }
    for (int j = 0; j < ngroups; j++) {
        const int last = min(C4_PER * (j + LEAD) + C4_PER - 1, ntiles - 1);
        const int issued = min(C4_P + C4_PER * j, ntiles);
        c4_wait_tiles_after<IPT>(issued - 1 - last);
        tile_barrier();
        for (int t = 0; t < C4_PER; t++) {
            const int i = C4_P + C4_PER * j + t;
            if (i < ntiles) issue(i);
        }
    }
}

// V producer P (0..3): per tile, positions 16P..16P+15 of the 16-dim slice.
// VT: one contiguous KB of the tiled copy, lane -> positions 16P + 4*(lane/16)
// ..+3 of dim lane%16, which is the consumer's LDS layout as it stands.
// Rows: lane -> position 16P + lane/4, dims 4*(lane%4)..+3 of the cache row
// (ring slots wrap).
template <int P, bool VT>
__device__ void c4_vproducer(const AttnExactArgs &A, Chain4Lds &L, int s0, int ctx, int h, int slice) {
    const int lane = threadIdx.x & 63;
    const int ntiles = (ctx + EX_TILE - 1) / EX_TILE;
    const char *v_base = (const char *)(A.v + (size_t)h * A.vd + slice * 16) + (lane & 3) * 16;
    const char *vt_base =
        VT ? (const char *)(A.vt + vt4_off((int64_t)h * A.vd + slice * 16, s0 + 16 * P, A.vt_stride)) + lane * 16
           : nullptr;
    const uint32_t row_bytes = (uint32_t)A.value_stride * 4u;
    const uint32_t wrap = (uint32_t)A.slot_count * row_bytes;
    const uint32_t step = 64u * row_bytes;
    uint32_t roff = (uint32_t)((s0 + 16 * P + (lane >> 2)) % A.slot_count) * row_bytes;
    auto issue = [&](int i) {
        const int sl = i & (C4_NT - 1);
        // streamed: the last tile holds the current position's V, stored by
        // a scores workgroup of this launch
        const bool fresh = A.sync != nullptr && i == ntiles - 1;
        if (fresh) stream_wait(A, h, i);
        const char *src = VT ? vt_base + (size_t)i * 4096u : v_base + roff;
        if (fresh) dma16_coherent(src, &L.v[sl][P * 256]);
        else dma16(src, &L.v[sl][P * 256]);
        if (!VT) {
            roff += step;
            if (roff >= wrap) roff -= wrap;
        }
    };
    c4_producer_loop<1, 0>(ntiles, issue);
}

// Scores producer: per tile the four heads' scores (lane -> head g0 +
// lane/16, positions 4*(lane%16)..+3; rows past kv_mul repeat the last head).
__device__ void c4_sproducer(const AttnExactArgs &A, Chain4Lds &L, int ctx, int h, int g0) {
    const int lane = threadIdx.x & 63, kvm = A.kv_mul;
    const int ntiles = (ctx + EX_TILE - 1) / EX_TILE;
    const int r = min(g0 + (lane >> 4), kvm - 1);
    const char *base = (const char *)(A.scores + (size_t)(h * kvm + r) * A.cap) + (lane & 15) * 16;
    int ready = 0;  // tiles known to be published (streamed launch)
    auto issue = [&](int i) {
        if (A.sync) {
            stream_wait_prefix(A, h, i, ntiles, ready);
            dma16_coherent(base + (uint32_t)i * 256u, &L.s[i & (C4_NT - 1)][0]);
        } else {
            dma16(base + (uint32_t)i * 256u, &L.s[i & (C4_NT - 1)][0]);
        }
    };
    c4_producer_loop<1, 1>(ntiles, issue);
}

// Coefficient wave k: row k of the ring (head g0 + k, or the last head of
// the group past kv_mul), the work of attn_exact_coef_kernel in position
// order, so the running max of the earlier tiles is carried instead of
// gathered: lane = position; the running max before each step is max(sink,
// earlier tiles, in-tile prefix), the step's coefficient and new-max bit as
// there.  (max is exact in any order and ignores NaN, so the values are the
// same; the sign of a zero maximum cannot change any comparison or
// coefficient.)  A group's four tiles are worked together (only the carried
// maximum is serial), group j + 1 between barriers j and j + 1, group 0
// before barrier 0; expf reads its table from LDS.
__device__ __forceinline__ void c4_egroup(const AttnExactArgs &A, Chain4Lds &L, int ctx, int ntiles, int i0, int k,
                                          float sink, float &mt) {
    const int lane = threadIdx.x & 63;
    float sc[C4_PER], p[C4_PER], run[C4_PER];
    bool valid[C4_PER];
#pragma unroll
    for (int t = 0; t < C4_PER; t++) {
        // tiles past the range read a slot they never write (no effect)
        sc[t] = L.s[(i0 + t) & (C4_NT - 1)][k * EX_TILE + lane];
        valid[t] = (i0 + t) * EX_TILE + lane < ctx;
    }
#pragma unroll
    for (int t = 0; t < C4_PER; t++) {
        // inclusive prefix max over lanes, the steps of dpp_max as single
        // v_max_f32_dpp instructions (a lane without a source keeps its value)
        float q = valid[t] ? sc[t] : -INFINITY;
        asm("s_nop 1\n\t"
            "v_max_f32_dpp %0, %0, %0 row_shr:1 row_mask:0xf bank_mask:0xf\n\t"
            "s_nop 1\n\t"
            "v_max_f32_dpp %0, %0, %0 row_shr:2 row_mask:0xf bank_mask:0xf\n\t"
            "s_nop 1\n\t"
            "v_max_f32_dpp %0, %0, %0 row_shr:4 row_mask:0xf bank_mask:0xf\n\t"
            "s_nop 1\n\t"
            "v_max_f32_dpp %0, %0, %0 row_shr:8 row_mask:0xf bank_mask:0xf\n\t"
            "s_nop 1\n\t"
            "v_max_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
            "s_nop 1\n\t"
            "v_max_f32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf"
            : "+v"(q));
        p[t] = q;
    }
#pragma unroll
    for (int t = 0; t < C4_PER; t++) {
        // each lane's exclusive prefix from lane - 1 (wave_shr:1), after the
        // running max of the tiles before
        const float prev = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, p[t]),
                                                                                 __builtin_bit_cast(int, p[t]), 0x138,
                                                                                 0xF, 0xF, false));
        const float m = A.sinks ? fmaxf(sink, mt) : mt;
        run[t] = lane == 0 ? m : fmaxf(m, prev);
        mt = fmaxf(mt, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p[t]), 63)));
    }
#pragma unroll
    for (int t = 0; t < C4_PER; t++) {
        const bool flag = valid[t] && sc[t] > run[t];
        const float x = flag ? run[t] - sc[t] : sc[t] - run[t];
        const float ex = expf_glibc_tab(x, L.exp2tab);
        const bool zero = (flag && !__builtin_isfinite(run[t])) || (!flag && !valid[t]);
        const float e = zero ? 0.0f : ex;
        const unsigned long long bits = __ballot(flag);
        if (i0 + t < ntiles) {
            const int sl = (i0 + t) & (C4_NT - 1);
            L.e[sl][k * EX_TILE + lane] = e;
            if (lane < 2) L.m[sl][2 * k + lane] = (uint32_t)(bits >> (32 * lane));
        }
    }
}
__device__ void c4_ewave(const AttnExactArgs &A, Chain4Lds &L, int ctx, int h, int g0, int k) {
    const int lane = threadIdx.x & 63, kvm = A.kv_mul;
    const int ntiles = (ctx + EX_TILE - 1) / EX_TILE;
    const int ngroups = (ntiles + C4_PER - 1) / C4_PER;
    const int head = h * kvm + min(g0 + k, kvm - 1);
    const float sink = A.sinks ? A.sinks[head] : 0.0f;
    if (k == 0 && lane < 32) L.exp2tab[lane] = kExp2fTab[lane];
    float mt = -INFINITY;  // max score of the tiles before
    RH_WAIT_LGKM0();
    tile_barrier();  // group 0's scores have landed; the table is in LDS
    c4_egroup(A, L, ctx, ntiles, 0, k, sink, mt);
    for (int j = 0; j < ngroups; j++) {
        RH_WAIT_LGKM0();  // this group's coefficients are in LDS before its barrier
        tile_barrier();
        if (C4_PER * (j + 1) < ntiles) c4_egroup(A, L, ctx, ntiles, C4_PER * (j + 1), k, sink, mt);
    }
}

// A wave with nothing to do still takes part in every barrier.
__device__ void c4_idle(int ctx) {
    const int ntiles = (ctx + EX_TILE - 1) / EX_TILE;
    const int ngroups = (ntiles + C4_PER - 1) / C4_PER;
    tile_barrier();
    for (int j = 0; j < ngroups; j++) tile_barrier();
}

// 16 steps of a 16-dim row: e16 = coefficient of step (lane % 16) of this
// row's head, v[j] = V of step j at this lane's dim (broadcast across the
// four rows), or 1 for the denominators.
// V tile layouts in LDS: VT = false [position][16 dims] (vt = &v[dcol], one
// value per read); VT = true [position/4][16 dims][4 positions] (vt =
// &v[4*dcol], four steps of the lane's dim per 16-byte read).
template <bool DEN, bool VT>
__device__ __forceinline__ void c4_load16(const float *et, const float *vt, int k, int lane, float &e16, float *v) {
    e16 = et[k * 16 + (lane & 15)];
    if (VT && !DEN) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = *(const float4 *)(vt + (4 * k + q) * 64);
            v[4 * q] = f.x;
            v[4 * q + 1] = f.y;
            v[4 * q + 2] = f.z;
            v[4 * q + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = DEN ? 1.0f : vt[(k * 16 + j) * 16];
    }
}

// One 16-step chunk holding a new maximum, per step in its own form (rows
// whose flags are clear take the ordinary form throughout).
template <bool X4>
__device__ __forceinline__ void c4_steps16_slow(float e16, const float *v, float &o, uint32_t bits) {
    float e[16];
    bcast16_all(e16, e);
    chain_steps16_flags<false, X4>(e, v, o, bits);
}

// The last, partial chunk of a range: steps 0..n-1 (n < 16), each in its
// own form as chain_steps16_flags (xd: the grouped/denominator form on a new
// maximum), e of step j from lane j of the row.
__device__ __forceinline__ void steps16_partial(float e16, const float *v, float &o, uint32_t bits, int n,
                                                bool xd) {
    float e[16];
    bcast16_all(e16, e);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        if (j < n) {
            const float on = fmaf(e[j], v[j], o);
            const float ox = xd ? fmaf(v[j], 1.0f, o * e[j]) : fmaf(o, e[j], v[j]);
            o = ((bits >> j) & 1u) ? ox : on;
        }
    }
}

// New-max summary of a group for the wave's four rows.  w: lane l < 8*C4_PER
// holds new-max word l & 1 of row (l >> 1) & 3 in tile l >> 3 of the group
// (0 in the other lanes); bit l of lo (hi) is set when that word has a new
// maximum in its low (high) 16 positions.  Chunk k of tile t (16 positions)
// is word k >> 1, half k & 1: its bits are 0x55 << (8t + (k >> 1)) of lo or
// hi.
__device__ __forceinline__ void c4_group_ballots(uint32_t w, uint32_t &lo, uint32_t &hi) {
    lo = (uint32_t)__builtin_amdgcn_ballot_w64((w & 0xFFFFu) != 0u);
    hi = (uint32_t)__builtin_amdgcn_ballot_w64((w >> 16) != 0u);
}

// One tile (four 16-step chunks) of a consumer group in one of three forms:
// FAST 16 DPP FMAs per chunk; AFF per chunk the fast run unless a row holds
// a new maximum in it, then the grouped form o = fma(a, v, o*m) on every
// step, (a, m) from the coefficient and the row's new-max bit; FLAGS
// (scale_add heads) per chunk the fast run unless the chunk holds a new
// maximum, then each step in its own form.  Chunk k computes from register
// set k & 1 while chunk k + 1 (or chunk 0 of the group's next tile) loads
// into the other.
enum { C4_FAST = 0, C4_AFF = 1, C4_FLAGS = 2 };
template <bool X4, bool DEN, bool VT, int MODE>
__device__ __forceinline__ void c4_tile(const Chain4Lds &L, int i, int row, int dcol, int lane, bool has_next,
                                        uint32_t glo, uint32_t ghi, int t, float (&a)[2], float (&v)[2][16],
                                        float &o) {
    const int sl = i & (C4_NT - 1), sn = (i + 1) & (C4_NT - 1);
    const float *et = &L.e[sl][row * EX_TILE], *vt = &L.v[sl][VT ? 4 * dcol : dcol];
    const float *en = &L.e[sn][row * EX_TILE], *vn = &L.v[sn][VT ? 4 * dcol : dcol];
    uint32_t w0 = 0, w1 = 0;
    if (MODE != C4_FAST) {
        w0 = L.m[sl][2 * row];
        w1 = L.m[sl][2 * row + 1];
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int c = k & 1, n = c ^ 1;
        RH_WAIT_LGKM0();
        if (k < 3) c4_load16<DEN, VT>(et, vt, k + 1, lane, a[n], v[n]);
        else if (has_next) c4_load16<DEN, VT>(en, vn, 0, lane, a[n], v[n]);
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t wk = (k >> 1) ? w1 : w0;
        const uint32_t bits = (k & 1) ? (wk >> 16) : (wk & 0xFFFFu);
        if (MODE == C4_FAST) {
            cons_fma16_dpp(a[c], v[c], o);
        } else if (MODE == C4_AFF) {
            // the grouped form only on chunks where a row holds a new
            // maximum: elsewhere (a, m) = (e, 1) and the forms agree
            const uint32_t half = (k & 1) ? ghi : glo;
            if (half & (0x55u << (8 * t + (k >> 1)))) {
                float a16, m16;
                aff_pair16(a[c], bits, lane, a16, m16);
                cons_affine16_dpp(a16, m16, v[c], o);
            } else {
                cons_fma16_dpp(a[c], v[c], o);
            }
        } else {
            const uint32_t half = (k & 1) ? ghi : glo;
            if (half & (0x55u << (8 * t + (k >> 1)))) c4_steps16_slow<X4>(a[c], v[c], o, bits);
            else cons_fma16_dpp(a[c], v[c], o);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The first nt (1..C4_PER) tiles of a consumer group, all complete, each tile
// in the form its new-max summary calls for (PART = false: all C4_PER, the
// count a constant).
template <bool X4, bool DEN, bool VT, bool PART>
__device__ __forceinline__ void c4_group(const Chain4Lds &L, int i0, int row, int dcol, int lane, float &o,
                                         int nt_part) {
    const int nt = PART ? nt_part : C4_PER;
    // the group's new-max words first, then chunk 0, so the summary is ready
    // while chunk 0 is still in flight
    const uint32_t wraw = lane < 8 * nt ? L.m[(i0 + (lane >> 3)) & (C4_NT - 1)][lane & 7] : 0u;
    const int s0 = i0 & (C4_NT - 1);
    float a[2], v[2][16];
    c4_load16<DEN, VT>(&L.e[s0][row * EX_TILE], &L.v[s0][VT ? 4 * dcol : dcol], 0, lane, a[0], v[0]);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t glo, ghi;
    c4_group_ballots(wraw, glo, ghi);
    const uint32_t any = glo | ghi;  // bits 8t..8t+7: tile t of the group
    if (any == 0u) {
        // no new maximum in any of the group's steps (the common case past
        // the first tiles): straight-line FMA runs
#pragma unroll
        for (int t = 0; t < C4_PER; t++)
            if (t < nt)
                c4_tile<X4, DEN, VT, C4_FAST>(L, i0 + t, row, dcol, lane, t + 1 < nt, glo, ghi, t, a, v, o);
    } else if (X4 || DEN) {
        // grouped form: the 16-step chunks of a tile holding a new maximum
        // for any of the four rows run o = fma(a, v, o*m) on every step
#pragma unroll
        for (int t = 0; t < C4_PER; t++) {
            if (t >= nt) break;
            if ((any >> (8 * t)) & 0xFFu)
                c4_tile<X4, DEN, VT, C4_AFF>(L, i0 + t, row, dcol, lane, t + 1 < nt, glo, ghi, t, a, v, o);
            else
                c4_tile<X4, DEN, VT, C4_FAST>(L, i0 + t, row, dcol, lane, t + 1 < nt, glo, ghi, t, a, v, o);
        }
    } else {
        // scale_add heads: each 16-step chunk holding a new maximum runs
        // every step in its own form
#pragma unroll
        for (int t = 0; t < C4_PER; t++)
            if (t < nt)
                c4_tile<X4, DEN, VT, C4_FLAGS>(L, i0 + t, row, dcol, lane, t + 1 < nt, glo, ghi, t, a, v, o);
    }
}

// The recurrence of one wave: DEN = false the outputs (lane = value dim of
// its row's head), DEN = true the denominators, the same recurrence with
// v = 1 (fma(e, 1, d) = d + e; on a new maximum fma(1, 1, d*e) = d*e + 1,
// the x4 form), starting from 1 with sinks; no V is read.
// PF: the complete tiles of a partial group in the chunked forms too (the
// separate chain launch; in the streamed launch the second instance of the
// group code would not fit the ten waves' registers)
template <bool X4, bool DEN, bool VT, bool PF>
__device__ void c4_consumer(const AttnExactArgs &A, Chain4Lds &L, int ctx, float *dst) {
    const int lane = threadIdx.x & 63, row = lane >> 4, dcol = lane & 15;
    const int ntiles = (ctx + EX_TILE - 1) / EX_TILE;
    const int ngroups = (ntiles + C4_PER - 1) / C4_PER;
    float o = (DEN && A.sinks) ? 1.0f : 0.0f;
    tile_barrier();
    for (int j = 0; j < ngroups; j++) {
        tile_barrier();
        const int i0 = C4_PER * j;
        const bool full = i0 + C4_PER <= ntiles && ctx >= (i0 + C4_PER) * EX_TILE;
        if (full) {
            c4_group<X4, DEN, VT, false>(L, i0, row, dcol, lane, o, C4_PER);
        } else {
            // (PF) the complete tiles in the chunked forms, then the rest
            // step by step
            int nfull = 0;
            if constexpr (PF) {
                while (nfull < C4_PER && i0 + nfull < ntiles && ctx >= (i0 + nfull + 1) * EX_TILE) nfull++;
                if (nfull > 0) c4_group<X4, DEN, VT, true>(L, i0, row, dcol, lane, o, nfull);
            }
            for (int i = i0 + nfull; i < min(i0 + C4_PER, ntiles); i++) {
                const int sl = i & (C4_NT - 1);
                const int ntok = min(EX_TILE, ctx - i * EX_TILE);
                const float *vt = &L.v[sl][dcol];
                const float *et = &L.e[sl][row * EX_TILE];
                const uint32_t mw0 = L.m[sl][2 * row], mw1 = L.m[sl][2 * row + 1];
                for (int t = 0; t < ntok; t++) {
                    const uint32_t mw = t < 32 ? mw0 : mw1;
                    const float e = et[t];
                    const float v = DEN ? 1.0f : (VT ? L.v[sl][(t >> 2) * 64 + 4 * dcol + (t & 3)] : vt[t * 16]);
                    const float on = fmaf(e, v, o);
                    const float ox = X4 ? fmaf(v, 1.0f, o * e) : fmaf(o, e, v);
                    o = ((mw >> (t & 31)) & 1u) ? ox : on;
                }
            }
        }
        RH_WAIT_LGKM0();  // this group's LDS reads are done before its slots are reused
    }
    if (dst) *dst = o;
}

// The output recurrence with V widened from bf16 cache rows in global memory
// (a bf16 cache whose range the tiled f32 copy cannot serve: an unaligned
// start or a wrapped ring), step by step, coefficients and new-max words
// from the ring as in c4_consumer.  Rare and slow; the V producers idle.
template <bool X4>
__device__ void c4_consumer_vg(const AttnExactArgs &A, Chain4Lds &L, int s0, int ctx, int h, int slice,
                               float *dst) {
    const int lane = threadIdx.x & 63, row = lane >> 4, dcol = lane & 15;
    const int ntiles = (ctx + EX_TILE - 1) / EX_TILE;
    const int ngroups = (ntiles + C4_PER - 1) / C4_PER;
    const uint16_t *vcol = (const uint16_t *)A.v + (size_t)h * A.vd + slice * 16 + dcol;
    float o = 0.0f;
    tile_barrier();
    for (int j = 0; j < ngroups; j++) {
        tile_barrier();
        for (int i = C4_PER * j; i < min(C4_PER * j + C4_PER, ntiles); i++) {
            const int sl = i & (C4_NT - 1);
            const int ntok = min(EX_TILE, ctx - i * EX_TILE);
            if (A.sync && i == ntiles - 1) {
                // streamed: the current position's V row is stored in this launch
                stream_wait(A, h, i);
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            }
            const float *et = &L.e[sl][row * EX_TILE];
            const uint32_t mw0 = L.m[sl][2 * row], mw1 = L.m[sl][2 * row + 1];
            for (int t = 0; t < ntok; t++) {
                const uint32_t mw = t < 32 ? mw0 : mw1;
                const float e = et[t];
                const int slot = (s0 + i * EX_TILE + t) % A.slot_count;
                const float v = bf16_to_f32(vcol[(size_t)kv_row(A, slot) * A.value_stride]);
                const float on = fmaf(e, v, o);
                const float ox = X4 ? fmaf(v, 1.0f, o * e) : fmaf(o, e, v);
                o = ((mw >> (t & 31)) & 1u) ? ox : on;
            }
        }
        RH_WAIT_LGKM0();
    }
    if (dst) *dst = o;
}

// grid: n_kv * ceil(kv_mul/4) * (vd/16) chain workgroups, then n_kv *
// ceil(kv_mul/4) denominator workgroups (the four heads' denominators as the
// same DPP recurrence with v = 1, no V); block b serves kv head b % n_kv.
// Waves: 0 the recurrence; 1, 2, 3, 5 the coefficient waves of rows 0-3; 9
// the scores producer; 4, 8, 6, 7 the V producers 0-3 (idle in denominator
// workgroups).  A workgroup's waves go to its four SIMDs in turn, so the
// recurrence wave shares its SIMD only with two V producers, which issue
// loads and hardly any VALU work.
#define C4_WAVES 10
__device__ __forceinline__ int c4_ewave_row(int wave) {
    return wave == 1 ? 0 : wave == 2 ? 1 : wave == 3 ? 2 : wave == 5 ? 3 : -1;
}
__device__ __forceinline__ int c4_vwave_part(int wave) {
    return wave == 4 ? 0 : wave == 8 ? 1 : wave == 6 ? 2 : wave == 7 ? 3 : -1;
}
__device__ __forceinline__ int chain4_blocks(const AttnExactArgs &A) {
    return A.n_kv * ((A.kv_mul + 3) / 4) * (A.vd / 16 + 1);
}
template <bool PF>
__device__ __forceinline__ void chain4_block(const AttnExactArgs &A, int block) {
    __shared__ Chain4Lds L;
    int s0, e0;
    exact_range(A, s0, e0);
    const int ctx = e0 - s0 + 1;
    if (ctx <= 0) return;
    const int kvm = A.kv_mul, ngrp = (kvm + 3) / 4, nsl = A.vd / 16;
    const int h = block % A.n_kv, r = block / A.n_kv;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    // V from the tiled transposed copy when the range starts on a multiple
    // of 4 positions, does not wrap, and its tiles stay inside the copy
    const int ntiles = (ctx + EX_TILE - 1) / EX_TILE;
    const bool vt_ok = A.vt != nullptr && (s0 & 3) == 0 && e0 < A.slot_count && s0 + ntiles * EX_TILE <= A.vt_stride;
    const bool vg = A.kv_bf16 && !vt_ok;  // bf16 rows cannot be streamed into the f32 ring as they are
    const bool den = r >= ngrp * nsl;
    const int g0 = den ? 4 * (r - ngrp * nsl) : 4 * (r / nsl), slice = den ? 0 : r % nsl;
    const int g = g0 + (lane >> 4);
    const int erow = c4_ewave_row(wave), vpart = c4_vwave_part(wave);
    if (erow >= 0) {
        c4_ewave(A, L, ctx, h, g0, erow);
    } else if (wave == 9) {
        c4_sproducer(A, L, ctx, h, g0);
    } else if (den) {
        if (wave == 0) c4_consumer<true, true, false, PF>(A, L, ctx, (g < kvm && (lane & 15) == 0) ? A.den + h * kvm + g : nullptr);
        else c4_idle(ctx);
    } else if (wave == 0) {
        float *dst = g < kvm ? A.out + (size_t)(h * kvm + g) * A.vd + slice * 16 + (lane & 15) : nullptr;
        const bool x4 = A.sinks == nullptr && (kvm == 4 || kvm == 6) && g0 == 0;
        if (vg) {
            if (x4) c4_consumer_vg<true>(A, L, s0, ctx, h, slice, dst);
            else c4_consumer_vg<false>(A, L, s0, ctx, h, slice, dst);
        } else if (vt_ok) {
            if (x4) c4_consumer<true, false, true, PF>(A, L, ctx, dst);
            else c4_consumer<false, false, true, PF>(A, L, ctx, dst);
        } else {
            if (x4) c4_consumer<true, false, false, PF>(A, L, ctx, dst);
            else c4_consumer<false, false, false, PF>(A, L, ctx, dst);
        }
    } else if (vg) {
        c4_idle(ctx);
    } else if (vt_ok) {
        if (vpart == 0) c4_vproducer<0, true>(A, L, s0, ctx, h, slice);
        else if (vpart == 1) c4_vproducer<1, true>(A, L, s0, ctx, h, slice);
        else if (vpart == 2) c4_vproducer<2, true>(A, L, s0, ctx, h, slice);
        else c4_vproducer<3, true>(A, L, s0, ctx, h, slice);
    } else {
        if (vpart == 0) c4_vproducer<0, false>(A, L, s0, ctx, h, slice);
        else if (vpart == 1) c4_vproducer<1, false>(A, L, s0, ctx, h, slice);
        else if (vpart == 2) c4_vproducer<2, false>(A, L, s0, ctx, h, slice);
        else c4_vproducer<3, false>(A, L, s0, ctx, h, slice);
    }
}

__global__ __launch_bounds__(64 * C4_WAVES) void attn_exact_chain4_kernel(AttnExactArgs A0) {
    const AttnExactArgs A = tok_view(A0);
    chain4_block<true>(A, blockIdx.x);
}

// A, B and C of one decode step in one launch, sized so every workgroup is
// resident at once: blocks 0..ns-1 are the scores workgroups, J = ns / n_kv
// per kv head, workgroup j scoring tiles j, j + J, j + 2J, ... in order, so
// the early tiles come first; the chain workgroups come last and compute
// while the later tiles are still being scored.  Only chain workgroups wait,
// each for a flag (see stream_wait), and the scores workgroups never do.
// The last workgroup to finish advances the epoch and resets the ticket for
// the next launch.
template <int HD>
__global__ __launch_bounds__(64 * C4_WAVES) void attn_exact_stream_kernel(AttnExactArgs A0) {
    AttnExactArgs A = A0;
    A.ep = __hip_atomic_load(A0.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int ns = (int)gridDim.x - chain4_blocks(A);
    if ((int)blockIdx.x >= ns) {
        chain4_block<false>(A, (int)blockIdx.x - ns);
        __syncthreads();
    } else {
        if (threadIdx.x >= 256) return;  // the scores work takes four waves
        const int J = ns / A.n_kv, j = (int)blockIdx.x / A.n_kv, h = (int)blockIdx.x - j * A.n_kv;
        for (int tile = j; tile < A.cap / EX_TILE; tile += J) {
            const bool wrote = scores8_tile<HD>(A, tile, h);
            if (!wrote) break;  // past the range (uniform)
            // this wave's device-scope stores (scores, f32 K/V rows)
            // complete; a bf16 cache's rows are plain stores and need the L2
            // written back
            if (A.kv_bf16) __threadfence();
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();  // also: the tile's LDS is free for the next
            if (threadIdx.x == 0)
                __hip_atomic_store(stream_flag(A, h, tile), A.ep + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (A.pf) {
            // workgroup i of a launch runs on XCD i % 8, in this launch and in
            // the GEMV's, so the row groups g with g % 8 == this XCD are the
            // ones its workgroups will compute there: one load per 128-byte
            // line of them, spread over this XCD's scores workgroups, while the
            // recurrences still run
            const int x = (int)blockIdx.x & 7, nx = (ns - x + 7) >> 3, ib = (int)blockIdx.x >> 3;
            const int ngr = (A.pf_rows + A.pf_group_rows - 1) / A.pf_group_rows;
            const int64_t gbytes = (int64_t)A.pf_group_rows * A.pf_stride;
            uint32_t acc = 0;
            for (int gi = x + 8 * ib; gi < ngr; gi += 8 * nx) {
                const uint8_t *base = A.pf + gi * gbytes;
                const int64_t nbytes = min(gbytes, (int64_t)(A.pf_rows - gi * A.pf_group_rows) * A.pf_stride);
                for (int64_t off = 128 * (int64_t)threadIdx.x; off < nbytes; off += 128 * 256)
                    acc ^= *(const uint32_t *)(base + off);
            }
            asm volatile("" ::"v"(acc));  // the loads stay; their values are not used
        }
    }
    if (threadIdx.x == 0) {
        // (nothing of this launch is read after the ticket but the epoch,
        // which the next launch reads)
        const uint32_t t = atomicAdd(A.sync + 1, 1u);
        if (t == gridDim.x - 1) {
            __hip_atomic_store(A.sync + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(A.sync, A.ep + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// C for many query tokens at once (prefill: grid z = token): a token's
// recurrence is short (its own position), so the launch is bound by
// throughput, not by one chain's latency.  Each wave is one independent task
// (token, kv head, group of four query heads, 16 value dims) or the group's
// denominators, with no LDS ring: V comes straight from the cache (the
// transposed copy gives four steps of a lane's dim per 16-byte load), the
// coefficients and new-max words from global memory, and many
// waves per SIMD hide the latency.  The update forms are the chain4
// consumer's, step for step.
// One chain of attn_exact_chain_tok_kernel: V from the transposed copy
// (MODE 1), from f32 cache rows (MODE 2) or bf16 ones (MODE 3), or v = 1 for
// the denominator (MODE 0).  Chunk k + 1's coefficient word, new-max bits and V values are
// loaded before chunk k's steps (two register sets, clamped indices, every
// load unconditional and straight-line), so a wave waits for one load round
// trip per launch rather than one per 16 steps.
template <int MODE>
__device__ __forceinline__ float chain_tok_run(const AttnExactArgs &A, int s0, int ctx, const float *ef,
                                               const uint32_t *mk, const float *vtr, int dim, bool x4, int lane,
                                               int dcol, float o) {
    constexpr bool DEN = MODE == 0;
    const int nk = (ctx + 15) / 16;
    auto load = [&](int k, float &e16, uint32_t &bits, float *v) {
        k = min(k, nk - 1);
        e16 = ef[16 * k + dcol];
        bits = (mk[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
        if constexpr (MODE == 0) {
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = 1.0f;
        } else if constexpr (MODE == 1) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                // four consecutive slots of the lane's dim: 64 floats per slot group
                const float4 f = *(const float4 *)(vtr + (size_t)(4 * k + q) * 64);
                v[4 * q] = f.x;
                v[4 * q + 1] = f.y;
                v[4 * q + 2] = f.z;
                v[4 * q + 3] = f.w;
            }
        } else {
            const int n = min(16, ctx - 16 * k);
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int slot = (s0 + 16 * k + min(j, n - 1)) % A.slot_count;
                const size_t vr = (size_t)kv_row(A, slot) * A.value_stride + dim;
                v[j] = MODE == 3 ? bf16_to_f32(((const uint16_t *)A.v)[vr]) : A.v[vr];
            }
        }
    };
    auto step = [&](int k, float e16, uint32_t bits, const float *v) {
        const int n = min(16, ctx - 16 * k);
        if (n == 16) {
            const uint32_t f = bits ? 1u : 0u;
            const uint32_t any = __builtin_amdgcn_readlane(f, 0) | __builtin_amdgcn_readlane(f, 16) |
                                 __builtin_amdgcn_readlane(f, 32) | __builtin_amdgcn_readlane(f, 48);
            if (any == 0u) {
                cons_fma16_dpp(e16, v, o);
            } else if (x4 || DEN) {
                float a16, m16;
                aff_pair16(e16, bits, lane, a16, m16);
                cons_affine16_dpp(a16, m16, v, o);
            } else {
                c4_steps16_slow<false>(e16, v, o, bits);
            }
        } else {
            steps16_partial(e16, v, o, bits, n, x4 || DEN);  // the last, partial chunk
        }
    };
    float ea, eb, va[16], vb[16];
    uint32_t ba, bb;
    load(0, ea, ba, va);
    for (int k = 0; k < nk; k += 2) {
        load(k + 1, eb, bb, vb);
        step(k, ea, ba, va);
        if (k + 1 >= nk) break;
        load(k + 2, ea, ba, va);
        step(k + 1, eb, bb, vb);
    }
    return o;
}

__global__ __launch_bounds__(256) void attn_exact_chain_tok_kernel(AttnExactArgs A0) {
    const AttnExactArgs A = tok_view(A0);
    int s0, e0;
    exact_range(A, s0, e0);
    const int ctx = e0 - s0 + 1;
    const int kvm = A.kv_mul, ngrp = (kvm + 3) / 4, nsl = A.vd / 16;
    const int n_chain = A.n_kv * ngrp * nsl, n_task = n_chain + A.n_kv * ngrp;
    const int task = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (ctx <= 0 || task >= n_task) return;
    const bool den = task >= n_chain;
    const int r = den ? task - n_chain : task;
    const int h = r % A.n_kv, rr = r / A.n_kv;
    const int g0 = 4 * (den ? rr : rr / nsl), slice = den ? 0 : rr % nsl;
    const int lane = threadIdx.x & 63, row = lane >> 4, dcol = lane & 15;
    const int g = g0 + row, gr = min(g, kvm - 1);
    const bool x4 = A.sinks == nullptr && (kvm == 4 || kvm == 6) && g0 == 0;
    const float *ef = A.e + e_index(A, h, gr, 0);
    const uint32_t *mk = A.newmask + (size_t)(h * kvm + gr) * (A.cap / 32);
    const int dim = h * A.vd + slice * 16 + dcol;
    const bool vt = A.vt != nullptr && (s0 & 3) == 0 && e0 < A.slot_count &&
                    s0 + (ctx + EX_TILE - 1) / EX_TILE * EX_TILE <= A.vt_stride;
    const float *vtr = vt ? A.vt + vt4_off(dim, s0, A.vt_stride) : nullptr;
    float o = (den && A.sinks) ? 1.0f : 0.0f;
    if (den) o = chain_tok_run<0>(A, s0, ctx, ef, mk, nullptr, dim, x4, lane, dcol, o);
    else if (vt) o = chain_tok_run<1>(A, s0, ctx, ef, mk, vtr, dim, x4, lane, dcol, o);
    else if (A.kv_bf16) o = chain_tok_run<3>(A, s0, ctx, ef, mk, nullptr, dim, x4, lane, dcol, o);
    else o = chain_tok_run<2>(A, s0, ctx, ef, mk, nullptr, dim, x4, lane, dcol, o);
    if (g < kvm) {
        if (den) {
            if (dcol == 0) A.den[h * kvm + g] = o;
        } else {
            A.out[(size_t)(h * kvm + g) * A.vd + slice * 16 + dcol] = o;
        }
    }
}

// Eight steps of four independent chains o_t += e_t(step) * v(step) with
// each e_t's step j from lane j of its 16-lane row (DPP row_newbcast), the
// chains interleaved so that the four FMAs of a step issue back to back.
#define FMA8X4_STEP(J, V)                                                                             \
    "v_fmac_f32_dpp %0, %4, " V " row_newbcast:" J " row_mask:0xf bank_mask:0xf\n\t"                  \
    "v_fmac_f32_dpp %1, %5, " V " row_newbcast:" J " row_mask:0xf bank_mask:0xf\n\t"                  \
    "v_fmac_f32_dpp %2, %6, " V " row_newbcast:" J " row_mask:0xf bank_mask:0xf\n\t"                  \
    "v_fmac_f32_dpp %3, %7, " V " row_newbcast:" J " row_mask:0xf bank_mask:0xf\n\t"
__device__ __forceinline__ void cons_fma8x4_dpp_lo(const float (&e)[4], const float *v, float (&o)[4]) {
    asm("s_nop 1\n\t" FMA8X4_STEP("0", "%8") FMA8X4_STEP("1", "%9") FMA8X4_STEP("2", "%10") FMA8X4_STEP("3", "%11")
            FMA8X4_STEP("4", "%12") FMA8X4_STEP("5", "%13") FMA8X4_STEP("6", "%14") FMA8X4_STEP("7", "%15")
        : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3])
        : "v"(e[0]), "v"(e[1]), "v"(e[2]), "v"(e[3]), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]),
          "v"(v[5]), "v"(v[6]), "v"(v[7]));
}
__device__ __forceinline__ void cons_fma8x4_dpp_hi(const float (&e)[4], const float *v, float (&o)[4]) {
    asm("s_nop 1\n\t" FMA8X4_STEP("8", "%8") FMA8X4_STEP("9", "%9") FMA8X4_STEP("10", "%10")
            FMA8X4_STEP("11", "%11") FMA8X4_STEP("12", "%12") FMA8X4_STEP("13", "%13") FMA8X4_STEP("14", "%14")
                FMA8X4_STEP("15", "%15")
        : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3])
        : "v"(e[0]), "v"(e[1]), "v"(e[2]), "v"(e[3]), "v"(v[8]), "v"(v[9]), "v"(v[10]), "v"(v[11]),
          "v"(v[12]), "v"(v[13]), "v"(v[14]), "v"(v[15]));
}
#undef FMA8X4_STEP

// A raw buffer resource over p: no stride, the largest record count (the
// callers keep every offset in range themselves), 32-bit data format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, 0x7fffffff, 0x00020000);
}

// C for four consecutive query tokens at once (prefill with a shared range
// start: no window, a linear cache and its tiled transposed V copy): each
// wave is attn_exact_chain_tok_kernel's task for tokens 4 Z .. 4 Z + 3 (grid
// z = Z), four chains per lane.  A chunk of V (four 16-byte loads per lane)
// serves the four tokens, each with its own coefficient word and new-max
// bits; chunk k + 1's loads are issued before chunk k's steps.  Chunks that
// every token runs whole without a new maximum take the interleaved DPP
// chains; others run each token's chain in its own form, exactly as the
// one-token kernel, so every token's output and denominator are its values.
__global__ __launch_bounds__(256) void attn_exact_chain_tok4_kernel(AttnExactArgs A) {
    constexpr int NT = 4;
    // the longest ranges (the last tokens) are dispatched first
    const int z0 = (int)(gridDim.z - 1 - blockIdx.z) * NT, nt = min(NT, A.n_tok - z0);
    const int s0 = A.start_t;
    const int ctx0 = A.pos0 + z0 - s0 + 1;  // the first token's range; token i's is ctx0 + i
    const int kvm = A.kv_mul, ngrp = (kvm + 3) / 4, nsl = A.vd / 16;
    const int n_chain = A.n_kv * ngrp * nsl, n_task = n_chain + A.n_kv * ngrp;
    const int task = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (nt <= 0 || ctx0 <= 0 || task >= n_task) return;
    const bool den = task >= n_chain;
    const int r = den ? task - n_chain : task;
    const int h = r % A.n_kv, rr = r / A.n_kv;
    const int g0 = 4 * (den ? rr : rr / nsl), slice = den ? 0 : rr % nsl;
    const int lane = threadIdx.x & 63, row = lane >> 4, dcol = lane & 15;
    const int g = g0 + row, gr = min(g, kvm - 1);
    const bool x4 = A.sinks == nullptr && (kvm == 4 || kvm == 6) && g0 == 0;
    // Every load is a buffer load: a wave-uniform resource and byte offset
    // (scalar registers) plus a lane's 32-bit byte offset, so that a chunk's
    // loads need no vector address registers and the next chunk's loads never
    // wait on this one's.  Token i's scratch is i * tok_scratch floats past
    // the first token's (tokens past the launch's end repeat its last).
    const __amdgpu_buffer_rsrc_t re = buf_rsrc(A.e + (int64_t)z0 * A.tok_scratch);
    const __amdgpu_buffer_rsrc_t rm = buf_rsrc(A.newmask + (int64_t)z0 * A.tok_scratch);
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(A.vt + vt4_off(h * A.vd + slice * 16, s0, A.vt_stride));
    int ctx[NT], tofs[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) {
        ctx[i] = ctx0 + min(i, nt - 1);
        tofs[i] = min(i, nt - 1) * (int)A.tok_scratch * 4;
    }
    const int off_e = ((int)e_index(A, h, gr, 0) + dcol) * 4;
    const int off_m = (h * kvm + gr) * (A.cap / 32) * 4, off_v = dcol * 16;
    const int nk = (ctx[NT - 1] + 15) / 16;  // chunks of the longest range
    float o[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) o[i] = (den && A.sinks) ? 1.0f : 0.0f;
    auto load = [&](auto dc, int k, float (&e16)[NT], uint32_t (&bits)[NT], float *v) {
        constexpr bool DEN = decltype(dc)::value;
        k = min(k, nk - 1);
#pragma unroll
        for (int i = 0; i < NT; i++) {
            const int ki = min(k, (ctx[i] + 15) / 16 - 1);  // a chunk past a token's range is not used
            e16[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(re, off_e, tofs[i] + 64 * ki, 0));
            // the word; step takes chunk k's half
            bits[i] = __builtin_amdgcn_raw_buffer_load_b32(rm, off_m, tofs[i] + 4 * (ki >> 1), 0);
        }
        if constexpr (DEN) {
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = 1.0f;
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                // four consecutive slots of the lane's dim: 64 floats per slot group
                const auto f = __builtin_amdgcn_raw_buffer_load_b128(rv, off_v, (4 * k + q) * 256, 0);
                v[4 * q] = __uint_as_float(f[0]);
                v[4 * q + 1] = __uint_as_float(f[1]);
                v[4 * q + 2] = __uint_as_float(f[2]);
                v[4 * q + 3] = __uint_as_float(f[3]);
            }
        }
    };
    // one token's 16-or-fewer steps of chunk k in its own form (the one-token
    // kernel's step)
    auto step1 = [&](int k, int i, float e16, uint32_t bits, const float *v) {
        const int n = min(16, ctx[i] - 16 * k);
        if (n <= 0) return;
        if (n == 16) {
            const uint32_t f = bits ? 1u : 0u;
            const uint32_t any = __builtin_amdgcn_readlane(f, 0) | __builtin_amdgcn_readlane(f, 16) |
                                 __builtin_amdgcn_readlane(f, 32) | __builtin_amdgcn_readlane(f, 48);
            if (any == 0u) {
                cons_fma16_dpp(e16, v, o[i]);
            } else if (x4 || den) {
                float a16, m16;
                aff_pair16(e16, bits, lane, a16, m16);
                cons_affine16_dpp(a16, m16, v, o[i]);
            } else {
                c4_steps16_slow<false>(e16, v, o[i], bits);
            }
        } else {
            steps16_partial(e16, v, o[i], bits, n, x4 || den);
        }
    };
    auto step = [&](int k, const float (&e16)[NT], const uint32_t (&words)[NT], const float *v) {
        uint32_t bits[NT], f = 0u;
#pragma unroll
        for (int i = 0; i < NT; i++) {
            bits[i] = (words[i] >> (16 * (k & 1))) & 0xFFFFu;  // chunk k of a token whose range holds it
            f |= bits[i];
        }
        // (a row's lanes hold the same words)
        const bool any = __builtin_amdgcn_ballot_w64(f != 0u) != 0u;
        if (!any && 16 * k + 16 <= ctx[0]) {
            // every token runs the whole chunk, none with a new maximum
            cons_fma8x4_dpp_lo(e16, v, o);
            cons_fma8x4_dpp_hi(e16, v, o);
        } else {
#pragma unroll
            for (int i = 0; i < NT; i++) step1(k, i, e16[i], bits[i], v);
        }
    };
    // the pipeline in two copies, the denominators' (v = 1, no V loads) and
    // the outputs', so that each copy's load waits count only its own loads
    auto run = [&](auto dc) {
        float ea[NT], eb[NT], va[16], vb[16];
        uint32_t ba[NT], bb[NT];
        load(dc, 0, ea, ba, va);
        for (int k = 0; k < nk; k += 2) {
            load(dc, k + 1, eb, bb, vb);
            step(k, ea, ba, va);
            if (k + 1 >= nk) break;
            load(dc, k + 2, ea, ba, va);
            step(k + 1, eb, bb, vb);
        }
    };
    if (den) run(std::true_type{});
    else run(std::false_type{});
    if (g < kvm) {
#pragma unroll
        for (int i = 0; i < NT; i++) {
            if (i >= nt) break;
            const int64_t zo = (int64_t)(z0 + i);
            if (den) {
                if (dcol == 0) A.den[zo * A.tok_scratch + h * kvm + g] = o[i];
            } else {
                A.out[zo * A.o_tok + (size_t)(h * kvm + g) * A.vd + slice * 16 + dcol] = o[i];
            }
        }
    }
}

// C (any layout): one wave per (query head, 64 value dims), grid (n_heads,
// ceil(vd/64)); V read straight from the cache, 32 steps per batch.  The
// denominator runs in every lane beside the output; slice 0 stores it.
__global__ __launch_bounds__(64) void attn_exact_chain_kernel(AttnExactArgs A0) {
    const AttnExactArgs A = tok_view(A0);
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
            const size_t vr = (size_t)kv_row(A, slot) * A.value_stride;
            vb[j] = A.kv_bf16 ? bf16_to_f32(((const uint16_t *)A.v)[(size_t)h * A.vd + (dim_ok ? dim : 0) + vr])
                              : vbase[vr];
            eb[j] = ef[t];
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
