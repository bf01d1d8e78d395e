// attention.hip — split-K flash-decode GQA attention over an f32 KV cache.
//
// Semantics follow the reference scan (online_attention*, src/model.rs:
// 5739-6198): positions t = start_t ..= end_t are read from ring slot
// t % slot_count (this equals the reference's incrementing-slot walk in both
// the linear and the wrapping case, including ranges longer than the ring,
// which revisit slots), scores are dot(q, k) * scale, and an optional sink
// logit joins the softmax with a zero value row (model.rs:5754-5755).
//
// Pass 1 (attn_partial): workgroup (chunk c, kv head h) scans one contiguous
// chunk of the range for all kv_mul query heads of h, so each K/V row is read
// from HBM once per token (GQA reuse), and writes (m, l, o) per head.
// Pass 2 (attn_combine): log-sum-exp merge of the chunks (+ sink), written as
// f32 and, optionally, as the Q8_K activation the next projection consumes.
#pragma once
#include "common.hpp"

namespace rh {

#define ATT_MAX_KVMUL 8
#define ATT_CHUNK_MAX 256

struct AttnArgs {
    const float *q;       // [n_heads * hd]
    const float *k;       // cache: slot s, kv head h at k + s*key_stride + h*hd
    const float *v;       // cache: v + s*value_stride + h*vd
    const float *sinks;   // [n_heads] or null
    float *part;          // [n_kv][n_chunks][kv_mul][vd + 2]
    float *out;           // [n_heads * vd]
    XQ xq;                // optional Q8_K of out (xq.qs == null: skip)
    const StepState *st;  // optional: positions come from the device
    int32_t n_heads, n_kv, kv_mul, hd, vd;
    int64_t key_stride, value_stride;
    int32_t slot_count;
    int32_t start_t, end_t;  // used when st == null
    int32_t window;          // with st: start = max(0, pos+1-window) if window>0 else 0
    int32_t n_chunks;
    float scale;
};

__device__ __forceinline__ void attn_range(const AttnArgs &A, int &start_t, int &end_t) {
    if (A.st) {
        end_t = A.st->pos;
        start_t = A.window > 0 ? max(0, end_t + 1 - A.window) : 0;
    } else {
        start_t = A.start_t;
        end_t = A.end_t;
    }
}

// HD = head dim (key), VD = value dim; both multiples of 4, <= 256.  A chunk
// of any length is scanned in sub-chunks of ATT_CHUNK_MAX positions with a
// running max / denominator, so no position is ever dropped.
template <int HD, int VD, int KVMUL>
__global__ __launch_bounds__(256) void attn_partial_kernel(AttnArgs A) {
    constexpr int LPT = HD / 4;         // lanes per token for the score pass
    constexpr int TPW = 64 / LPT;       // tokens per wave step (score pass)
    constexpr int LPV = VD / 4;         // lanes per token for the value pass
    constexpr int TPV = 64 / LPV;
    __shared__ float s_p[KVMUL][ATT_CHUNK_MAX];
    __shared__ float s_o[4][KVMUL][VD];
    __shared__ float s_run[KVMUL][3];  // running max, running denominator, rescale

    const int c = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps tile math scalar
    int start_t, end_t;
    attn_range(A, start_t, end_t);
    const int ctx = end_t - start_t + 1;
    int chunk = (ctx + A.n_chunks - 1) / A.n_chunks;
    if (chunk < 16) chunk = 16;
    const int t0 = start_t + c * chunk;
    const int t1 = min(end_t + 1, t0 + chunk);
    float *part = A.part + ((size_t)h * A.n_chunks + c) * KVMUL * (VD + 2);
    if (ctx <= 0 || t0 >= t1) {
        if (tid < KVMUL) {
            part[tid * (VD + 2) + VD] = -INFINITY;
            part[tid * (VD + 2) + VD + 1] = 0.0f;
        }
        return;
    }

    const int sub = lane / LPT, dl = lane % LPT;
    const int vsub = lane / LPV, vl = lane % LPV;
    float4 qv[KVMUL];
#pragma unroll
    for (int g = 0; g < KVMUL; g++) qv[g] = *(const float4 *)(A.q + (size_t)(h * KVMUL + g) * HD + dl * 4);
    float4 acc[KVMUL];
#pragma unroll
    for (int g = 0; g < KVMUL; g++) acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tid < KVMUL) {
        s_run[tid][0] = -INFINITY;
        s_run[tid][1] = 0.0f;
    }

    for (int s0 = t0; s0 < t1; s0 += ATT_CHUNK_MAX) {
        const int n = min(ATT_CHUNK_MAX, t1 - s0);
        // ---- scores ----------------------------------------------------------
        for (int base = wave * TPW; base < n; base += 4 * TPW) {
            int tl = base + sub;
            bool ok = tl < n;
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f);
            if (ok) {
                int slot = (s0 + tl) % A.slot_count;
                kv = *(const float4 *)(A.k + (size_t)slot * A.key_stride + (size_t)h * HD + dl * 4);
            }
            float dot[KVMUL];
#pragma unroll
            for (int g = 0; g < KVMUL; g++) {
                float d = qv[g].x * kv.x;
                d = fmaf(qv[g].y, kv.y, d);
                d = fmaf(qv[g].z, kv.z, d);
                d = fmaf(qv[g].w, kv.w, d);
                if (LPT >= 2) d += swz_xor<1>(d);
                if (LPT >= 4) d += swz_xor<2>(d);
                if (LPT >= 8) d += swz_xor<4>(d);
                if (LPT >= 16) d += swz_xor<8>(d);
                if (LPT >= 32) d += swz_xor<16>(d);
                if (LPT >= 64) d += __shfl_xor(d, 32, 64);
                dot[g] = d;
            }
            if (ok && dl == 0) {
#pragma unroll
                for (int g = 0; g < KVMUL; g++) s_p[g][tl] = dot[g] * A.scale;
            }
        }
        __syncthreads();
        // ---- running softmax statistics, one wave per head -----------------
        for (int g = wave; g < KVMUL; g += 4) {
            float m = -INFINITY;
            for (int i = lane; i < n; i += 64) m = fmaxf(m, s_p[g][i]);
            m = wave_max(m);
            float m_old = s_run[g][0];
            float m_new = fmaxf(m_old, m);
            float l = 0.0f;
            for (int i = lane; i < n; i += 64) {
                float p = expf(s_p[g][i] - m_new);
                s_p[g][i] = p;
                l += p;
            }
            l = wave_sum(l);
            if (lane == 0) {
                float alpha = m_old == -INFINITY ? 0.0f : expf(m_old - m_new);
                s_run[g][0] = m_new;
                s_run[g][1] = s_run[g][1] * alpha + l;
                s_run[g][2] = alpha;
            }
        }
        __syncthreads();
        // ---- weighted values --------------------------------------------------
#pragma unroll
        for (int g = 0; g < KVMUL; g++) {
            float al = s_run[g][2];
            acc[g].x *= al;
            acc[g].y *= al;
            acc[g].z *= al;
            acc[g].w *= al;
        }
        for (int base = wave * TPV; base < n; base += 4 * TPV) {
            int tl = base + vsub;
            if (tl < n) {
                int slot = (s0 + tl) % A.slot_count;
                float4 vv = *(const float4 *)(A.v + (size_t)slot * A.value_stride + (size_t)h * VD + vl * 4);
#pragma unroll
                for (int g = 0; g < KVMUL; g++) {
                    float p = s_p[g][tl];
                    acc[g].x = fmaf(p, vv.x, acc[g].x);
                    acc[g].y = fmaf(p, vv.y, acc[g].y);
                    acc[g].z = fmaf(p, vv.z, acc[g].z);
                    acc[g].w = fmaf(p, vv.w, acc[g].w);
                }
            }
        }
        __syncthreads();
    }
    // fold the TPV token groups of each wave, then the four waves
#pragma unroll
    for (int g = 0; g < KVMUL; g++) {
        for (int o = LPV; o < 64; o <<= 1) {
            acc[g].x += __shfl_xor(acc[g].x, o, 64);
            acc[g].y += __shfl_xor(acc[g].y, o, 64);
            acc[g].z += __shfl_xor(acc[g].z, o, 64);
            acc[g].w += __shfl_xor(acc[g].w, o, 64);
        }
        if (vsub == 0) *(float4 *)&s_o[wave][g][vl * 4] = acc[g];
    }
    __syncthreads();
    for (int i = tid; i < KVMUL * VD; i += 256) {
        int g = i / VD, d = i % VD;
        float o = (s_o[0][g][d] + s_o[1][g][d]) + (s_o[2][g][d] + s_o[3][g][d]);
        part[g * (VD + 2) + d] = o;
    }
    if (tid < KVMUL) {
        part[tid * (VD + 2) + VD] = s_run[tid][0];
        part[tid * (VD + 2) + VD + 1] = s_run[tid][1];
    }
}

// One workgroup per 256 output elements (a Q8_K block); thread = element.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs A) {
    __shared__ float red[4];
    const int e = blockIdx.x * 256 + threadIdx.x;
    const int total = A.n_heads * A.vd;
    float o = 0.0f;
    if (e < total) {
        int head = e / A.vd, d = e % A.vd;
        int h = head / A.kv_mul, g = head % A.kv_mul;
        const float *p0 = A.part + (size_t)h * A.n_chunks * A.kv_mul * (A.vd + 2) + (size_t)g * (A.vd + 2);
        const size_t cstride = (size_t)A.kv_mul * (A.vd + 2);
        float M = A.sinks ? A.sinks[head] : -INFINITY;
        for (int c = 0; c < A.n_chunks; c++) M = fmaxf(M, p0[c * cstride + A.vd]);
        float L = A.sinks ? expf(A.sinks[head] - M) : 0.0f;
        float acc = 0.0f;
        if (M != -INFINITY) {
            for (int c = 0; c < A.n_chunks; c++) {
                const float *pc = p0 + c * cstride;
                float l = pc[A.vd + 1];
                if (l > 0.0f) {
                    float w = expf(pc[A.vd] - M);
                    L = fmaf(w, l, L);
                    acc = fmaf(w, pc[d], acc);
                }
            }
        }
        o = L > 0.0f ? acc / L : 0.0f;
        A.out[e] = o;
    }
    if (A.xq.qs == nullptr) return;
    // Q8_K of this 256-block (total is a multiple of 256 when requested)
    float amax = block_max_256(fabsf(o), red);
    float dsc = amax * (1.0f / 127.0f);
    float id = amax > 0.0f ? 127.0f / amax : 0.0f;
    int q = (int)__builtin_rintf(o * id);
    q = max(-128, min(127, q));
    A.xq.qs[e] = (int8_t)q;
    if (threadIdx.x == 0) A.xq.d[blockIdx.x] = dsc;
    int s = q;
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    s += __shfl_xor(s, 8, 64);
    if ((threadIdx.x & 15) == 0) A.xq.sums16[e >> 4] = (int16_t)s;
    s += __shfl_xor(s, 16, 64);
    if ((threadIdx.x & 31) == 0) A.xq.bsums[e >> 5] = (int16_t)s;
}

}  // namespace rh
