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
#define ATT_TP 64  // positions per sub-tile of a split
#define ATT_CB 16  // partials a combine lane loads before merging them

// Floats per (split, query head) partial: vd outputs, then m and l, padded so
// every partial starts 16-byte aligned.
__host__ __device__ constexpr int att_pstride(int vd) { return vd + 4; }

struct AttnArgs {
    const float *q;       // [n_heads * hd]
    const float *k;       // cache: slot s, kv head h at k + s*key_stride + h*hd
    const float *v;       // cache: v + s*value_stride + h*vd
    const float *sinks;   // [n_heads] or null
    float *part;          // [n_kv][n_chunks][kv_mul][att_pstride(vd)]
    float *out;           // [n_heads * vd]
    XQ xq;                // optional Q8_K of out (xq.qs == null: skip)
    const StepState *st;  // optional: positions come from the device
    int32_t n_heads, n_kv, kv_mul, hd, vd;
    int64_t key_stride, value_stride;
    int32_t slot_count;
    int32_t start_t, end_t;  // used when st == null
    int32_t window;          // with st: start = max(0, pos+1-window) if window>0 else st->start_t
    int32_t n_chunks;
    float scale;
};

__device__ __forceinline__ void attn_range(const AttnArgs &A, int &start_t, int &end_t) {
    if (A.st) {
        end_t = A.st->pos;
        start_t = A.window > 0 ? max(0, end_t + 1 - A.window) : A.st->start_t;
    } else {
        start_t = A.start_t;
        end_t = A.end_t;
    }
}

// xor-1 / xor-2 lane exchange inside a quad (DPP quad_perm).
__device__ __forceinline__ float quad_xor1(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_xor2(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
}

// Pass 1: workgroup (split c, kv head h) covers `per` positions (a multiple
// of ATT_TP) of the range for all KVMUL query heads of h, so every K/V row
// is read from HBM once per token.  Per sub-tile of ATT_TP positions all of
// its K and V loads are issued first, each 64-lane load instruction reading
// whole 128-byte lines (K: 8 lanes per position, 32 positions per pass; V:
// TV lanes per row), then:
//   scores: the 8 lanes of a position split the head dim, q from LDS, the
//           partial dots summed across the 8 lanes;
//   softmax: tile max per head (wave shuffles + LDS), p = exp(s - m),
//            running (m, l) rescaled as in online softmax;
//   values: acc[g] += p * v with p broadcast from LDS.
// Outputs (m, l, o) per head; the combine merges the splits.
template <int HD, int KVMUL>
__global__ __launch_bounds__(256) void attn_partial_kernel(AttnArgs A) {
    constexpr int KF = HD / 32;        // float4 of a K row per lane (8 lanes per row)
    constexpr int NP = ATT_TP / 32;    // K passes (32 positions each)
    constexpr int QS = 4 * KF + 4;     // LDS stride of a lane's q slice (padded: slices hit distinct banks)
    constexpr int TV = HD / 4;         // threads per V row
    constexpr int PG = 256 / TV;       // V position groups
    constexpr int PPG = ATT_TP / PG;   // positions per V group
    constexpr int PS = att_pstride(HD);
    __shared__ __align__(16) float s_q[KVMUL][8][QS];
    __shared__ float s_p[KVMUL][ATT_TP];
    __shared__ float s_mx[4][KVMUL], s_sm[4][KVMUL];
    __shared__ __align__(16) float s_o[4][KVMUL][HD];

    const int c = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int start_t, end_t;
    attn_range(A, start_t, end_t);
    const int ctx = end_t - start_t + 1;
    const int per = ((ctx + A.n_chunks - 1) / A.n_chunks + ATT_TP - 1) / ATT_TP * ATT_TP;
    const int t0 = c * per, t1 = min(ctx, t0 + per);  // positions relative to start_t
    float *part = A.part + ((size_t)h * A.n_chunks + c) * KVMUL * PS;
    if (ctx <= 0 || t0 >= t1) {
        for (int i = tid; i < KVMUL * PS; i += 256) part[i] = (i % PS) == HD ? -INFINITY : 0.0f;
        return;
    }
    // lane j8 of a position holds dims (8i + j8)*4 .. +3, i < KF
    for (int i = tid; i < KVMUL * HD; i += 256) {
        const int g = i / HD, d = i % HD, f = d >> 2;
        s_q[g][f & 7][4 * (f >> 3) + (d & 3)] = A.q[(size_t)(h * KVMUL + g) * HD + d];
    }
    const int pk = tid >> 3, j8 = tid & 7;    // score pass: position within a pass, lane of the position
    const int d4 = tid % TV, pg = tid / TV;   // value pass: float4 column, position group
    const float *kb = A.k + (size_t)h * HD + 4 * j8;
    const float *vb = A.v + (size_t)h * HD + d4 * 4;
    float m_run[KVMUL], l_run[KVMUL];
    float4 acc[KVMUL];
#pragma unroll
    for (int g = 0; g < KVMUL; g++) {
        m_run[g] = -INFINITY;
        l_run[g] = 0.0f;
        acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    for (int s0 = t0; s0 < t1; s0 += ATT_TP) {
        float4 kr[NP][KF], vr[PPG];
#pragma unroll
        for (int r = 0; r < NP; r++) {
            const int slot = (start_t + min(s0 + 32 * r + pk, t1 - 1)) % A.slot_count;
            const float *kp = kb + (size_t)slot * A.key_stride;
#pragma unroll
            for (int i = 0; i < KF; i++) kr[r][i] = *(const float4 *)(kp + 32 * i);
        }
#pragma unroll
        for (int i = 0; i < PPG; i++) {
            const int sl = (start_t + min(s0 + pg * PPG + i, t1 - 1)) % A.slot_count;
            vr[i] = *(const float4 *)(vb + (size_t)sl * A.value_stride);
        }
        float sc[NP][KVMUL], tmx[KVMUL];
#pragma unroll
        for (int g = 0; g < KVMUL; g++) {
            float m = -INFINITY;
#pragma unroll
            for (int r = 0; r < NP; r++) {
                float d = 0.0f;
#pragma unroll
                for (int i = 0; i < KF; i++) {
                    const float4 qv = *(const float4 *)&s_q[g][j8][4 * i];
                    d = fmaf(qv.x, kr[r][i].x, d);
                    d = fmaf(qv.y, kr[r][i].y, d);
                    d = fmaf(qv.z, kr[r][i].z, d);
                    d = fmaf(qv.w, kr[r][i].w, d);
                }
                d += quad_xor1(d);
                d += quad_xor2(d);
                d += __shfl_xor(d, 4, 64);
                sc[r][g] = (s0 + 32 * r + pk < t1) ? d * A.scale : -INFINITY;
                m = fmaxf(m, sc[r][g]);
            }
            m = fmaxf(m, __shfl_xor(m, 8, 64));
            m = fmaxf(m, __shfl_xor(m, 16, 64));
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            tmx[g] = m;
        }
        if (lane == 0)
#pragma unroll
            for (int g = 0; g < KVMUL; g++) s_mx[wave][g] = tmx[g];
        __syncthreads();
        float alpha[KVMUL], psum[KVMUL];
#pragma unroll
        for (int g = 0; g < KVMUL; g++) {
            const float t = fmaxf(fmaxf(s_mx[0][g], s_mx[1][g]), fmaxf(s_mx[2][g], s_mx[3][g]));
            const float mn = fmaxf(m_run[g], t);
            alpha[g] = m_run[g] == -INFINITY ? 0.0f : __expf(m_run[g] - mn);
            m_run[g] = mn;
            float v = 0.0f;
#pragma unroll
            for (int r = 0; r < NP; r++) {
                const float pe = sc[r][g] == -INFINITY ? 0.0f : __expf(sc[r][g] - mn);
                if ((g & 7) == j8) s_p[g][32 * r + pk] = pe;
                v += j8 == 0 ? pe : 0.0f;
            }
            v += __shfl_xor(v, 8, 64);
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            psum[g] = v;
        }
        if (lane == 0)
#pragma unroll
            for (int g = 0; g < KVMUL; g++) s_sm[wave][g] = psum[g];
        __syncthreads();
#pragma unroll
        for (int g = 0; g < KVMUL; g++) {
            l_run[g] = l_run[g] * alpha[g] + ((s_sm[0][g] + s_sm[1][g]) + (s_sm[2][g] + s_sm[3][g]));
            acc[g].x *= alpha[g];
            acc[g].y *= alpha[g];
            acc[g].z *= alpha[g];
            acc[g].w *= alpha[g];
        }
#pragma unroll
        for (int i = 0; i < PPG; i++) {
            const int pos = pg * PPG + i;
#pragma unroll
            for (int g = 0; g < KVMUL; g++) {
                const float pp = s_p[g][pos];
                acc[g].x = fmaf(pp, vr[i].x, acc[g].x);
                acc[g].y = fmaf(pp, vr[i].y, acc[g].y);
                acc[g].z = fmaf(pp, vr[i].z, acc[g].z);
                acc[g].w = fmaf(pp, vr[i].w, acc[g].w);
            }
        }
        __syncthreads();  // s_p, s_mx and s_sm are rewritten by the next sub-tile
    }
    // fold the position groups: inside the wave, then the four waves
#pragma unroll
    for (int g = 0; g < KVMUL; g++) {
        for (int o = TV; o < 64; o <<= 1) {
            acc[g].x += __shfl_xor(acc[g].x, o, 64);
            acc[g].y += __shfl_xor(acc[g].y, o, 64);
            acc[g].z += __shfl_xor(acc[g].z, o, 64);
            acc[g].w += __shfl_xor(acc[g].w, o, 64);
        }
        if (lane < TV) *(float4 *)&s_o[wave][g][4 * d4] = acc[g];
    }
    __syncthreads();
    for (int i = tid; i < KVMUL * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        part[g * PS + d] = (s_o[0][g][d] + s_o[1][g][d]) + (s_o[2][g][d] + s_o[3][g][d]);
    }
    if (tid < KVMUL) {
        part[tid * PS + HD] = m_run[tid];
        part[tid * PS + HD + 1] = l_run[tid];
    }
}

// Online merge of one partial (m, l, o) into (M, L, acc).
__device__ __forceinline__ void att_merge(float &M, float &L, float4 &acc, float m, float l, float4 o) {
    if (m == -INFINITY) return;
    const float mn = fmaxf(M, m);
    const float a = M == -INFINITY ? 0.0f : __expf(M - mn);
    const float b = __expf(m - mn);
    L = L * a + l * b;
    acc.x = acc.x * a + o.x * b;
    acc.y = acc.y * a + o.y * b;
    acc.z = acc.z * a + o.z * b;
    acc.w = acc.w * a + o.w * b;
    M = mn;
}

// Pass 2: one workgroup per 256 outputs (a Q8_K block), lane = four outputs
// of one head, wave w = the splits c = w mod 4 (ATT_CB partials in flight per
// lane), then the four waves merged through LDS, the sink logit joining as a
// partial with l = 1 and a zero value row (model.rs:5754-5755).  Wave 0
// writes the f32 outputs and, when requested, their Q8_K quantization.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs A) {
    __shared__ float s_m[4][64], s_l[4][64];
    __shared__ float4 s_a[4][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int total = A.n_heads * A.vd, PS = att_pstride(A.vd);
    const int e0 = blockIdx.x * 256 + 4 * lane;
    const bool ok = e0 < total;
    const int head = ok ? e0 / A.vd : 0, d = e0 % A.vd;
    const int h = head / A.kv_mul, g = head % A.kv_mul;
    const size_t cst = (size_t)A.kv_mul * PS;
    const float *p0 = A.part + (size_t)h * A.n_chunks * cst + (size_t)g * PS;
    float M = -INFINITY, L = 0.0f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (wave == 0 && A.sinks && ok) {
        M = A.sinks[head];
        L = 1.0f;
    }
    for (int base = wave; base < A.n_chunks; base += 4 * ATT_CB) {
        float mm[ATT_CB], ll[ATT_CB];
        float4 oo[ATT_CB];
#pragma unroll
        for (int k = 0; k < ATT_CB; k++) {
            const int cc = min(base + 4 * k, A.n_chunks - 1);
            const float *pc = p0 + cc * cst;
            mm[k] = pc[A.vd];
            ll[k] = pc[A.vd + 1];
            oo[k] = *(const float4 *)(pc + d);
        }
#pragma unroll
        for (int k = 0; k < ATT_CB; k++)
            if (base + 4 * k < A.n_chunks) att_merge(M, L, acc, mm[k], ll[k], oo[k]);
    }
    s_m[wave][lane] = M;
    s_l[wave][lane] = L;
    s_a[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 1; w < 4; w++) att_merge(M, L, acc, s_m[w][lane], s_l[w][lane], s_a[w][lane]);
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    if (L > 0.0f) {
        const float inv = 1.0f / L;
        o = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    }
    if (ok) *(float4 *)(A.out + e0) = o;
    if (A.xq.qs == nullptr) return;
    // Q8_K of this 256-block (total is a multiple of 256 when requested)
    const float amax = wave_max(fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w))));
    const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
    const float ov[4] = {o.x, o.y, o.z, o.w};
    int qv[4], s = 0;
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        qv[i] = max(-128, min(127, (int)__builtin_rintf(ov[i] * id)));
        s += qv[i];
        packed |= (uint32_t)(qv[i] & 0xFF) << (8 * i);
    }
    *(uint32_t *)(A.xq.qs + e0) = packed;
    if (lane == 0) A.xq.d[blockIdx.x] = amax * (1.0f / 127.0f);
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    if ((lane & 3) == 0) A.xq.sums16[e0 >> 4] = (int16_t)s;
    s += __shfl_xor(s, 4, 64);
    if ((lane & 7) == 0) A.xq.bsums[e0 >> 5] = (int16_t)s;
}

}  // namespace rh
