// common.hpp — device helpers shared by the gfx950 kernels.
//
// Built with -ffp-contract=off: a*b+c stays two roundings unless a kernel
// calls fmaf() explicitly, which it does only where the reference uses an FMA
// intrinsic or where no reference rounding point is being reproduced.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define RH_WAVE 64

namespace rh {

// ---- byte-stream loads (block fields are only 1/2/4-byte aligned) --------
// memcpy keeps these well defined for any alignment; on gfx950 hipcc lowers a
// 16-byte copy to a single global_load_dwordx4.
__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
__device__ __forceinline__ uint2 ld8(const uint8_t *p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}
__device__ __forceinline__ uint32_t ld4(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}
__device__ __forceinline__ uint16_t ld2(const uint8_t *p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}

// Direct global -> LDS loads: lane l's 16 (or 4) bytes from its own address
// land at lds + 16 l (4 l); completion is counted by vmcnt.
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
// lgkmcnt(0) only
#define RH_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | (0 << 8) | (3 << 14))
// lgkmcnt(N) only (N <= 15)
#define RH_WAIT_LGKM(N) __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | ((N) << 8) | (3 << 14))

// IEEE half -> float (exact; v_cvt_f32_f16).
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// bf16 <-> f32 as the reference's f32_to_bf16 / bf16_to_f32 (src/simd.rs:
// 82-96): widening is exact; narrowing rounds to nearest even, a NaN keeps
// its payload with the quiet bit set.
__host__ __device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
}
__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float x) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    if (x != x) return (uint16_t)((b >> 16) | 0x0040u);
    return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}
// f32 with the value a bf16 store keeps
__host__ __device__ __forceinline__ float bf16_round(float x) { return bf16_to_f32(f32_to_bf16(x)); }
// four consecutive bf16 (8 bytes) widened
__device__ __forceinline__ float4 bf16x4_load(const uint16_t *p) {
    const uint2 u = *(const uint2 *)p;
    return make_float4(__builtin_bit_cast(float, u.x << 16), __builtin_bit_cast(float, u.x & 0xFFFF0000u),
                       __builtin_bit_cast(float, u.y << 16), __builtin_bit_cast(float, u.y & 0xFFFF0000u));
}
__device__ __forceinline__ float ldh(const uint8_t *p) { return h2f(ld2(p)); }

// v_dot4_i32_i8: c + sum_k a.byte[k] * b.byte[k] (signed bytes, exact).
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// ---- DPP / swizzle reductions ---------------------------------------------
// quad_perm controls: xor-1 = [1,0,3,2] = 0xB1, xor-2 = [2,3,0,1] = 0x4E.
__device__ __forceinline__ int quad_sum_i32(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
    v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
    return v;
}

// ds_swizzle bit mode within 32 lanes: offset = and_mask | or<<5 | xor<<10.
template <int XOR>
__device__ __forceinline__ float swz_xor(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x1F | (XOR << 10)));
}

__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
// max over the wave, in every lane: DPP shifts inside each 16-lane row
// leave the row's max in its lane 15, row_bcast:15 and :31 carry rows 0-1 and
// 2-3 into lane 63 (a lane with no source keeps its own value).  Max is exact
// in any order.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_max(float v) {
    const int o = __builtin_bit_cast(int, v);
    return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(o, o, CTRL, ROWS, 0xF, false)));
}
__device__ __forceinline__ float wave_max(float v) {
    v = dpp_max<0x111, 0xF>(v);  // row_shr:1
    v = dpp_max<0x112, 0xF>(v);  // row_shr:2
    v = dpp_max<0x114, 0xF>(v);  // row_shr:4
    v = dpp_max<0x118, 0xF>(v);  // row_shr:8
    v = dpp_max<0x142, 0xA>(v);  // row_bcast:15
    v = dpp_max<0x143, 0xC>(v);  // row_bcast:31
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Within each 16-lane row, every lane gets the row's max / integer sum:
// quad_perm xor 1 and xor 2, then row_ror 4 and 8 (all sources valid).
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, dpp_i<0xB1>(__builtin_bit_cast(int, v))));
    v = fmaxf(v, __builtin_bit_cast(float, dpp_i<0x4E>(__builtin_bit_cast(int, v))));
    v = fmaxf(v, __builtin_bit_cast(float, dpp_i<0x124>(__builtin_bit_cast(int, v))));
    v = fmaxf(v, __builtin_bit_cast(float, dpp_i<0x128>(__builtin_bit_cast(int, v))));
    return v;
}
__device__ __forceinline__ int row_sum16_i(int v) {
    v += dpp_i<0xB1>(v);
    v += dpp_i<0x4E>(v);
    v += dpp_i<0x124>(v);
    v += dpp_i<0x128>(v);
    return v;
}
__device__ __forceinline__ int wave_sum_i32(int v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Block-wide (256 threads = 4 waves) reductions through LDS; every thread
// receives the same value, computed in the same order on every block.
__device__ __forceinline__ float block_sum_256(float v, float *red) {
    v = wave_sum(v);
    int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    float r = (red[0] + red[1]) + (red[2] + red[3]);
    return r;
}
__device__ __forceinline__ float block_max_256(float v, float *red) {
    v = wave_max(v);
    int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// sum(x*x) in the exact order of dot_f32_avx2(x, x) (src/simd.rs:6547-6586):
// 32 lanes = four 8-wide FMA accumulators over 32-element chunks, combined as
// (acc0+acc1)+(acc2+acc3), then the 8-element tail chunks, the hsum_avx tree
// ((t0+t4)+(t1+t5)) + ((t2+t6)+(t3+t7)), then the scalar tail.  x is read
// from LDS (s_x, already staged); every workgroup computes the same value.
// red needs 33 floats.
__device__ float sumsq_avx2_order(const float *s_x, int n, float *red) {
    const int main32 = n / 32;
    if (threadIdx.x < 32) {
        const int L = threadIdx.x;
        float acc = 0.0f;
        int c = 0;
        for (; c + 8 <= main32; c += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = s_x[32 * (c + j) + L];
#pragma unroll
            for (int j = 0; j < 8; j++) acc = fmaf(v[j], v[j], acc);
        }
        for (; c < main32; c++) {
            float v = s_x[32 * c + L];
            acc = fmaf(v, v, acc);
        }
        red[L] = acc;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float t[8];
#pragma unroll
        for (int l = 0; l < 8; l++) t[l] = (red[l] + red[8 + l]) + (red[16 + l] + red[24 + l]);
        const int ts = main32 * 32, tail8 = (n - ts) / 8;
        for (int i = 0; i < tail8; i++)
#pragma unroll
            for (int l = 0; l < 8; l++) {
                float v = s_x[ts + 8 * i + l];
                t[l] = fmaf(v, v, t[l]);
            }
        float sum = ((t[0] + t[4]) + (t[1] + t[5])) + ((t[2] + t[6]) + (t[3] + t[7]));
        for (int i = ts + tail8 * 8; i < n; i++) sum += s_x[i] * s_x[i];
        red[32] = sum;
    }
    __syncthreads();
    float r = red[32];
    __syncthreads();
    return r;
}

// Q8_K activation buffers (device): int8 quants, per-256 f32 scale, per-32
// and per-16 int16 group sums.  The per-16 sums serve the Q6_K kernel's
// "-32" offset and are not part of the reference layout.
struct XQ {
    int8_t *qs;
    float *d;
    int16_t *bsums;
    int16_t *sums16;
};

// Decode step state kept on the device so a captured graph can replay every
// token without host updates.
// Float offset of value column j (kv head * vd + dim) at slot p in the tiled
// transposed V copy, layout [j / 16][p / 4][j % 16][p % 4] with vt_stride
// slots per column (a multiple of 4): the 16 dims of a slice over 64
// consecutive slots are one contiguous 4 KB block, and 16 bytes hold four
// consecutive slots of one dim.
__host__ __device__ __forceinline__ size_t vt4_off(int64_t j, int64_t p, int64_t vt_stride) {
    return (size_t)(((j >> 4) * (vt_stride >> 2) + (p >> 2)) * 64 + (j & 15) * 4 + (p & 3));
}

struct StepState {
    int32_t pos;       // position being written / attended to (end_t)
    int32_t start_t;   // first attended position
    int32_t token;     // current input token (device-token mode)
    int32_t n_recent;  // valid entries in recent[]
    int32_t recent[64];
};

}  // namespace rh
