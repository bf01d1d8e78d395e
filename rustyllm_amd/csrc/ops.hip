// ops.hip — the small per-token ops fused around the GEMVs and attention.
#pragma once
#include "common.hpp"

namespace rh {

// Q8_K of one 256-block held one element per thread (256 threads):
// d = amax * (1/127), q = clamp(rne(x * (127/amax))), group sums per 16/32
// (quantize_row_q8k_scalar/avx2, src/simd.rs:5013-5101).  1/127 and 127/amax
// are correctly rounded (hipcc's default f32 division), rne is v_rndne_f32.
__device__ __forceinline__ void q8k_block_store(float v, int blk, int e, XQ xq, float *red) {
    float amax = block_max_256(fabsf(v), red);
    float id = amax > 0.0f ? 127.0f / amax : 0.0f;
    int q = (int)__builtin_rintf(v * id);
    q = max(-128, min(127, q));
    xq.qs[e] = (int8_t)q;
    if (threadIdx.x == 0) xq.d[blk] = amax * (1.0f / 127.0f);
    // integer sums (exact in any order): per 16 lanes, then rows 0+1 and 2+3
    int s = row_sum16_i(q);
    if ((threadIdx.x & 15) == 0) xq.sums16[e >> 4] = (int16_t)s;
    const int lane = threadIdx.x & 63;
    const int r1 = __builtin_amdgcn_readlane(s, 16), r3 = __builtin_amdgcn_readlane(s, 48);
    s += lane < 32 ? r1 : r3;
    if ((threadIdx.x & 31) == 0) xq.bsums[e >> 5] = (int16_t)s;
}

__global__ __launch_bounds__(256) void quantize_q8k_kernel(const float *x, int n, XQ xq) {
    __shared__ float red[4];
    int e = blockIdx.x * 256 + threadIdx.x;
    float v = e < n ? x[e] : 0.0f;
    q8k_block_store(v, blockIdx.x, e, xq, red);
}

// RMSNorm (rms_norm_into, src/model.rs:5429-5437): ss = sum(x^2)/n,
// scale = 1/sqrt(ss + eps), out = (x*scale)*w, with the sum in the
// reference's order (so scale, and everything after it, matches bit for
// bit).  x is first staged in LDS by all threads at once (dynamic LDS of n
// floats).  Each block then writes its 256 outputs and, when xq.qs != null
// and n % 256 == 0, their Q8_K quantization.
// One row's RMSNorm (element blockIdx.x * 256 + threadIdx.x) and its Q8_K
// block; every workgroup of the row computes the row's sum.
__device__ __forceinline__ void rmsnorm_row(const float *x, const float *w, float eps, int n, float *xn, XQ xq) {
    extern __shared__ float s_x[];
    __shared__ float red[40];
    {
        // loads eight float4 per thread at a time, all issued before their
        // stores (clamped unconditional loads: conditionally loaded array
        // elements were kept in scratch)
        const int n4 = n >> 2, tid = threadIdx.x;
        for (int k0 = 0; 256 * k0 < n4; k0 += 8) {
            float4 t[8];
#pragma unroll
            for (int k = 0; k < 8; k++) t[k] = ((const float4 *)x)[min(tid + 256 * (k0 + k), n4 - 1)];
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (tid + 256 * (k0 + k) < n4) ((float4 *)s_x)[tid + 256 * (k0 + k)] = t[k];
        }
        for (int i = 4 * n4 + tid; i < n; i += 256) s_x[i] = x[i];
    }
    __syncthreads();
    float ss = sumsq_avx2_order(s_x, n, red);
    float scale = 1.0f / sqrtf(ss / (float)n + eps);
    int e = blockIdx.x * 256 + threadIdx.x;
    float o = 0.0f;
    if (e < n) {
        o = s_x[e] * scale * w[e];
        if (xn) xn[e] = o;
    }
    if (xq.qs) q8k_block_store(o, blockIdx.x, e, xq, red);
}

__global__ __launch_bounds__(256) void rmsnorm_q8k_kernel(const float *x, const float *w, float eps, int n,
                                                          float *xn, XQ xq) {
    rmsnorm_row(x, w, eps, n, xn, xq);
}

// RoPE + KV store (apply_rope_qk / apply_rope_qk_neox, src/model.rs:
// 5562-5647; KVCache::write_k/v :1478-1502).  cos/sin come from a table the
// host built with libm sinf/cosf of (float)pos * inv_freq[i], exactly the
// reference's angle, so rotated values match bit for bit.  The slot is pos,
// or pos % slots for a ring (slot_for_pos, src/model.rs:1458-1464).
struct RopeArgs {
    float *q;             // [n_heads*hd], rotated in place
    const float *k;       // [n_kv*hd]
    const float *v;       // [n_kv*vd]
    float *kcache;        // layer K cache [slots][n_kv*hd]
    float *vcache;        // layer V cache [slots][n_kv*vd]
    const float *cos_t;   // [max_pos][hd/2]
    const float *sin_t;
    const StepState *st;  // pos source when non-null
    int32_t pos;
    int32_t max_pos;      // rows of the cos/sin table
    int32_t n_heads, n_kv, hd, vd, slots, ring, neox;
    int32_t q_tok, k_tok, v_tok;  // per-token row strides of q/k/v (prefill: token blockIdx.y at pos + y)
    float *vtcache;       // optional tiled transposed V copy (vt4_off layout), or null
    int32_t vt_stride;
    int32_t kv_bf16;      // 1: kcache / vcache hold bf16 (uint16), narrowed as KVCache::write_k/v do;
                          // the f32 V copy then holds the widened bf16 values
    int32_t slot_off;     // with ring = 0: the row is pos - slot_off (a linear buffer starting there)
};

__global__ __launch_bounds__(256) void rope_kv_kernel(RopeArgs A) {
    const int z = blockIdx.y;
    const int pos = (A.st ? A.st->pos : A.pos) + z;
    A.q += (int64_t)z * A.q_tok;
    A.k += (int64_t)z * A.k_tok;
    A.v += (int64_t)z * A.v_tok;
    if (pos < 0 || pos >= A.max_pos) return;
    const int half = A.hd / 2;
    const int slot = A.ring ? pos % A.slots : pos - A.slot_off;
    const float *ct = A.cos_t + (size_t)pos * half;
    const float *stb = A.sin_t + (size_t)pos * half;
    const int nq = A.n_heads * half, nk = A.n_kv * half;
    const int kvd = A.n_kv * A.hd, vvd = A.n_kv * A.vd;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < nq + nk + vvd; i += gridDim.x * blockDim.x) {
        if (i < nq + nk) {
            bool isq = i < nq;
            int j = isq ? i : i - nq;
            int head = j / half, p = j % half;
            int i0, i1;
            if (A.neox) {
                i0 = head * A.hd + p;
                i1 = i0 + half;
            } else {
                i0 = head * A.hd + 2 * p;
                i1 = i0 + 1;
            }
            float c = ct[p], s = stb[p];
            const float *src = isq ? A.q : A.k;
            float v0 = src[i0], v1 = src[i1];
            float r0 = v0 * c - v1 * s;
            float r1 = v0 * s + v1 * c;
            if (isq) {
                A.q[i0] = r0;
                A.q[i1] = r1;
            } else if (A.kv_bf16) {
                uint16_t *kc = (uint16_t *)A.kcache + (size_t)slot * kvd;
                kc[i0] = f32_to_bf16(r0);
                kc[i1] = f32_to_bf16(r1);
            } else {
                float *kc = A.kcache + (size_t)slot * kvd;
                kc[i0] = r0;
                kc[i1] = r1;
            }
        } else {
            int j = i - nq - nk;
            float v = A.v[j];
            if (A.kv_bf16) {
                const uint16_t h = f32_to_bf16(v);
                ((uint16_t *)A.vcache)[(size_t)slot * vvd + j] = h;
                v = bf16_to_f32(h);
            } else {
                A.vcache[(size_t)slot * vvd + j] = v;
            }
            if (A.vtcache) A.vtcache[vt4_off(j, slot, A.vt_stride)] = v;
        }
    }
}

// Embedding row (token_embd.row_into, src/model.rs:267-289): dequantize row
// `token` (from the step state when st != null).
__constant__ float kLut4[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

__device__ float dequant_elem(const uint8_t *wr, int fmt, int e) {
    if (fmt == 0) {
        float f;
        __builtin_memcpy(&f, wr + 4 * e, 4);
        return f;
    }
    if (fmt == 8) {
        const uint8_t *blk = wr + (e >> 5) * 34;
        return ldh(blk) * (float)(int8_t)blk[2 + (e & 31)];
    }
    if (fmt == 12) {
        const uint8_t *blk = wr + (e >> 8) * 144;
        int p = e & 255, j = p >> 6, hi = (p >> 5) & 1, l = p & 31;
        int is = 2 * j + hi;
        const uint8_t *s = blk + 4;
        int sc, m;
        if (is < 4) {
            sc = s[is] & 63;
            m = s[is + 4] & 63;
        } else {
            sc = (s[is + 4] & 0xF) | ((s[is - 4] >> 6) << 4);
            m = (s[is + 4] >> 4) | ((s[is] >> 6) << 4);
        }
        float d1 = ldh(blk) * (float)sc, m1 = ldh(blk + 2) * (float)m;
        uint8_t byte = blk[16 + 32 * j + l];
        return d1 * (float)(hi ? (byte >> 4) : (byte & 0xF)) - m1;
    }
    if (fmt == 14) {
        const uint8_t *blk = wr + (e >> 8) * 210;
        int p = e & 255, n = p >> 7, pp = p & 127, k = pp >> 5, l = pp & 31;
        const uint8_t *ql = blk + 64 * n, *qh = blk + 128 + 32 * n;
        const int8_t *sc = (const int8_t *)(blk + 192 + 8 * n);
        uint8_t lo = (k & 1) ? ql[l + 32] : ql[l];
        int nib = (k & 2) ? (lo >> 4) : (lo & 0xF);
        int q = (nib | (((qh[l] >> (2 * k)) & 3) << 4)) - 32;
        return ldh(blk + 208) * (float)sc[l / 16 + 2 * k] * (float)q;
    }
    if (fmt == 39) {
        const uint8_t *blk = wr + (e >> 5) * 17;
        int p = e & 31;
        uint8_t byte = blk[p >> 1];
        uint32_t ex = blk[16];
        float s = ex == 0 ? __builtin_bit_cast(float, 0x00400000u) : __builtin_bit_cast(float, ex << 23);
        return kLut4[(p & 1) ? (byte >> 4) : (byte & 0xF)] * s;
    }
    return 0.0f;
}

__global__ void embed_kernel(const uint8_t *w, int64_t row_stride, int fmt, int dim, const StepState *st, int token,
                             float *x) {
    int tok = st ? st->token : token;
    const uint8_t *wr = w + (int64_t)tok * row_stride;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < dim; e += gridDim.x * blockDim.x)
        x[e] = dequant_elem(wr, fmt, e);
}

// Greedy pick (sample_with_scratch, src/sampling.rs:78-83): repeat penalty over
// the recent tokens in order, applied once per occurrence
// (apply_repeat_penalty :321-338), then the first maximum among finite logits
// (argmax_finite_token :341-356).  Stage 1: every block reduces a slice; the
// last block to finish (ticket counter, reset by that block) reduces the
// partials, writes the token, appends it to the recent window
// (push_recent_token, src/runtime.rs:514-521) and advances pos.
struct ArgmaxArgs {
    float *logits;
    int32_t n;
    float penalty;
    StepState *st;
    float *part_v;
    int32_t *part_i;
    uint32_t *ticket;
    int32_t *out_tokens;  // optional: out_tokens[out_index[0]++] = token
    int32_t *out_index;
    int32_t advance;      // 1: pos++ and token = winner
};

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

__global__ __launch_bounds__(256) void argmax_greedy_kernel(ArgmaxArgs A) {
    __shared__ int32_t s_rec[64];
    __shared__ int32_t s_nrec;
    __shared__ float s_v[256];
    __shared__ int32_t s_i[256];
    __shared__ bool s_last;
    const int tid = threadIdx.x;
    if (tid == 0) s_nrec = A.st ? A.st->n_recent : 0;
    if (tid < 64) s_rec[tid] = A.st ? A.st->recent[tid] : 0;
    __syncthreads();
    const int nrec = s_nrec;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    // the window in registers (uniform: scalar loads); each occurrence of a
    // token applies the penalty once more, and all apply the same map, so an
    // element needs only its occurrence count
    int rec[64];
#pragma unroll
    for (int r = 0; r < 64; r++) rec[r] = s_rec[r];
    for (int i = blockIdx.x * 256 + tid; i < A.n; i += gridDim.x * 256) {
        float v = A.logits[i];
        if (A.penalty != 1.0f) {
            int k = 0;
#pragma unroll
            for (int r = 0; r < 64; r++) k += (r < nrec && rec[r] == i) ? 1 : 0;
            for (int r = 0; r < k; r++) v = !isfinite(v) ? -INFINITY : (v > 0.0f ? v / A.penalty : v * A.penalty);
        }
        if (!isfinite(v)) v = -INFINITY;
        if (better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    s_v[tid] = bv;
    s_i[tid] = bi;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o && better(s_v[tid + o], s_i[tid + o], s_v[tid], s_i[tid])) {
            s_v[tid] = s_v[tid + o];
            s_i[tid] = s_i[tid + o];
        }
        __syncthreads();
    }
    if (tid == 0) {
        // the partial by device-scope stores (through the XCD's non-coherent
        // L2), complete before the ticket, instead of a cache write-back fence
        __hip_atomic_store(A.part_v + blockIdx.x, s_v[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(A.part_i + blockIdx.x, s_i[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        uint32_t t = atomicAdd(A.ticket, 1u);
        s_last = (t == gridDim.x - 1);
    }
    __syncthreads();
    if (!s_last) return;
    bv = -INFINITY;
    bi = 0x7fffffff;
    for (int b = tid; b < (int)gridDim.x; b += 256) {
        float v = __hip_atomic_load(A.part_v + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int i = __hip_atomic_load(A.part_i + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    s_v[tid] = bv;
    s_i[tid] = bi;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o && better(s_v[tid + o], s_i[tid + o], s_v[tid], s_i[tid])) {
            s_v[tid] = s_v[tid + o];
            s_i[tid] = s_i[tid + o];
        }
        __syncthreads();
    }
    int tok = s_i[0];
    if (tok == 0x7fffffff) tok = 0;  // all logits non-finite: token 0, as the reference
    if (tid == 0) {
        *A.ticket = 0;
        if (A.out_tokens) {
            int k = *A.out_index;
            A.out_tokens[k] = tok;
            *A.out_index = k + 1;
        }
    }
    if (A.st && A.advance) {
        // the window as read at the start (s_rec, s_nrec: nothing else writes
        // it during the launch), shifted by 64 threads at once when full
        StepState *st = A.st;
        if (nrec == 64) {
            if (tid < 64) st->recent[tid] = tid < 63 ? s_rec[tid + 1] : tok;
        } else if (tid == 0) {
            st->recent[nrec] = tok;
            st->n_recent = nrec + 1;
        }
        if (tid == 0) {
            st->token = tok;
            st->pos = st->pos + 1;
        }
    }
}

// Step-state helpers for the prefill loop: set token/pos from a device array.
__global__ void set_step_kernel(StepState *st, const int32_t *tokens, int idx, int pos, int push_recent) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    int tok = tokens[idx];
    st->token = tok;
    st->pos = pos;
    if (push_recent) {
        int nr = st->n_recent;
        if (nr == 64) {
            for (int r = 0; r < 63; r++) st->recent[r] = st->recent[r + 1];
            st->recent[63] = tok;
        } else {
            st->recent[nr] = tok;
            st->n_recent = nr + 1;
        }
    }
}

}  // namespace rh
