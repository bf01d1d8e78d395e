// synth.cpp — seeded synthetic weights and this repo's own GGUF block
// quantizers (host code, libsynth.so).
//
// The reference ships no weight quantizer (its tests hand-build block bytes),
// so these are written from the block format definitions that the reference's
// dequantizers read (src/simd.rs:4044-4294): Q8_0 (34 B / 32), Q4_K
// (144 B / 256), Q6_K (210 B / 256) and the reference's MXFP4 layout
// (17 B / 32: 16 nibble bytes, low nibble = element 2i, then one e8m0 byte).
// The CPU oracle and the GPU consume the same bytes, so the choice of
// quantizer cannot affect parity.
//
// Random numbers: row r of a tensor with seed s draws from xoshiro256**
// seeded by splitmix64(s, r), with Box-Muller normals, so the bytes do not
// depend on the thread count.
#include <immintrin.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

inline uint64_t splitmix64(uint64_t &x) {
    uint64_t z = (x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Xoshiro {
    uint64_t s[4];
    Xoshiro(uint64_t seed, uint64_t stream) {
        uint64_t x = seed * 0x2545F4914F6CDD1Dull + stream * 0x9E3779B97F4A7C15ull + 0x1234567ull;
        for (auto &v : s) v = splitmix64(x);
    }
    static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    inline uint64_t next() {
        uint64_t r = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
        s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3];
        s[2] ^= t; s[3] = rotl(s[3], 45);
        return r;
    }
    inline double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
};

inline void normal_row(uint64_t seed, uint64_t row, float stdv, float mean, float *out, int64_t n) {
    Xoshiro g(seed, row);
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = g.uniform(), u2 = g.uniform();
        double r = std::sqrt(-2.0 * std::log(u1));
        double a = 6.283185307179586 * u2;
        out[i] = (float)(mean + stdv * r * std::cos(a));
        if (i + 1 < n) out[i + 1] = (float)(mean + stdv * r * std::sin(a));
    }
}

inline uint16_t f32_to_f16(float x) { return (uint16_t)_cvtss_sh(x, 0); }
inline float f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }

inline int nearest_int(float x) { return (int)std::nearbyint(x); }

void quant_q8_0(const float *x, int64_t n, uint8_t *out) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float *xb = x + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(xb[i]));
        uint16_t dh = f32_to_f16(amax / 127.0f);
        float d = f16_to_f32(dh);
        float id = d > 0.0f ? 1.0f / d : 0.0f;
        uint8_t *o = out + b * 34;
        o[0] = (uint8_t)(dh & 0xff);
        o[1] = (uint8_t)(dh >> 8);
        for (int i = 0; i < 32; i++) o[2 + i] = (uint8_t)(int8_t)std::clamp(nearest_int(xb[i] * id), -127, 127);
    }
}

void quant_q4_k(const float *x, int64_t n, uint8_t *out) {
    for (int64_t b = 0; b < n / 256; b++) {
        const float *xb = x + b * 256;
        float scale[8], minv[8];
        for (int j = 0; j < 8; j++) {
            float mn = 0.0f, mx = 0.0f;
            for (int l = 0; l < 32; l++) {
                mn = std::min(mn, xb[32 * j + l]);
                mx = std::max(mx, xb[32 * j + l]);
            }
            scale[j] = (mx - mn) / 15.0f;
            minv[j] = -mn;
        }
        float ms = *std::max_element(scale, scale + 8), mm = *std::max_element(minv, minv + 8);
        uint16_t dh = f32_to_f16(ms / 63.0f), mh = f32_to_f16(mm / 63.0f);
        float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
        uint8_t sc[8], m[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = (uint8_t)std::clamp(d > 0 ? nearest_int(scale[j] / d) : 0, 0, 63);
            m[j] = (uint8_t)std::clamp(dmin > 0 ? nearest_int(minv[j] / dmin) : 0, 0, 63);
        }
        uint8_t *o = out + b * 144;
        o[0] = (uint8_t)(dh & 0xff); o[1] = (uint8_t)(dh >> 8);
        o[2] = (uint8_t)(mh & 0xff); o[3] = (uint8_t)(mh >> 8);
        uint8_t *s = o + 4;
        for (int j = 0; j < 4; j++) {
            s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
            s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
        }
        uint8_t q[256];
        for (int j = 0; j < 8; j++) {
            float dj = d * (float)sc[j], mj = dmin * (float)m[j];
            for (int l = 0; l < 32; l++) {
                int v = dj > 0 ? nearest_int((xb[32 * j + l] + mj) / dj) : 0;
                q[32 * j + l] = (uint8_t)std::clamp(v, 0, 15);
            }
        }
        uint8_t *qs = o + 16;
        for (int g = 0; g < 4; g++)
            for (int l = 0; l < 32; l++) qs[32 * g + l] = (uint8_t)(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
    }
}

void quant_q6_k(const float *x, int64_t n, uint8_t *out) {
    for (int64_t b = 0; b < n / 256; b++) {
        const float *xb = x + b * 256;
        float scale[16];
        float amax_s = 0.0f;
        for (int j = 0; j < 16; j++) {
            float amax = 0.0f;
            for (int l = 0; l < 16; l++) amax = std::max(amax, std::fabs(xb[16 * j + l]));
            scale[j] = amax / 31.0f;
            amax_s = std::max(amax_s, scale[j]);
        }
        uint16_t dh = f32_to_f16(amax_s / 127.0f);
        float d = f16_to_f32(dh);
        int8_t sc[16];
        uint8_t q[256];
        for (int j = 0; j < 16; j++) {
            sc[j] = (int8_t)std::clamp(d > 0 ? nearest_int(scale[j] / d) : 0, -128, 127);
            float dj = d * (float)sc[j];
            for (int l = 0; l < 16; l++) {
                int v = dj != 0.0f ? nearest_int(xb[16 * j + l] / dj) : 0;
                q[16 * j + l] = (uint8_t)(std::clamp(v, -32, 31) + 32);
            }
        }
        uint8_t *o = out + b * 210;
        uint8_t *ql = o, *qh = o + 128;
        for (int h = 0; h < 2; h++) {
            const uint8_t *qq = q + 128 * h;
            for (int l = 0; l < 32; l++) {
                ql[64 * h + l] = (uint8_t)((qq[l] & 0xF) | ((qq[64 + l] & 0xF) << 4));
                ql[64 * h + 32 + l] = (uint8_t)((qq[32 + l] & 0xF) | ((qq[96 + l] & 0xF) << 4));
                qh[32 * h + l] = (uint8_t)((qq[l] >> 4) | ((qq[32 + l] >> 4) << 2) | ((qq[64 + l] >> 4) << 4) |
                                           ((qq[96 + l] >> 4) << 6));
            }
        }
        std::memcpy(o + 192, sc, 16);
        o[208] = (uint8_t)(dh & 0xff);
        o[209] = (uint8_t)(dh >> 8);
    }
}

const float kE2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

void quant_mxfp4(const float *x, int64_t n, uint8_t *out) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float *xb = x + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(xb[i]));
        int e = 0;
        if (amax > 0.0f) e = (int)std::ceil(std::log2(amax / 6.0f));
        e = std::clamp(e, -127, 127);
        float inv = std::ldexp(1.0f, -e);
        uint8_t codes[32];
        for (int i = 0; i < 32; i++) {
            float v = std::fabs(xb[i]) * inv;
            int best = 0;
            float bd = 1e30f;
            for (int k = 0; k < 8; k++) {
                float dd = std::fabs(v - kE2M1[k]);
                if (dd < bd) { bd = dd; best = k; }
            }
            codes[i] = (uint8_t)(best | (xb[i] < 0.0f && best != 0 ? 8 : 0));
        }
        uint8_t *o = out + b * 17;
        for (int i = 0; i < 16; i++) o[i] = (uint8_t)(codes[2 * i] | (codes[2 * i + 1] << 4));
        o[16] = (uint8_t)(e + 127);
    }
}

int64_t row_bytes(int dtype, int64_t cols) {
    switch (dtype) {
    case 0: return cols * 4;
    case 8: return (cols / 32) * 34;
    case 12: return (cols / 256) * 144;
    case 14: return (cols / 256) * 210;
    case 39: return (cols / 32) * 17;
    default: return -1;
    }
}

void quant_row(int dtype, const float *x, int64_t n, uint8_t *out) {
    switch (dtype) {
    case 0: std::memcpy(out, x, (size_t)n * 4); break;
    case 8: quant_q8_0(x, n, out); break;
    case 12: quant_q4_k(x, n, out); break;
    case 14: quant_q6_k(x, n, out); break;
    case 39: quant_mxfp4(x, n, out); break;
    }
}

}  // namespace

extern "C" {

int64_t synth_row_bytes(int dtype, int64_t cols) { return row_bytes(dtype, cols); }

// Fills rows x cols f32 with N(mean, std) (row r uses stream r of `seed`).
void synth_normal_f32(uint64_t seed, int64_t rows, int64_t cols, float stdv, float mean, float *out) {
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t r = 0; r < rows; r++) normal_row(seed, (uint64_t)r, stdv, mean, out + r * cols, cols);
}

// Quantizes rows x cols f32 into GGUF blocks of `dtype` (GGML id).
int synth_quantize(int dtype, const float *x, int64_t rows, int64_t cols, uint8_t *out) {
    int64_t rb = row_bytes(dtype, cols);
    if (rb < 0) return 0;
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t r = 0; r < rows; r++) quant_row(dtype, x + r * cols, cols, out + r * rb);
    return 1;
}

// Generates N(0, std) rows and quantizes them in one pass (no full f32 copy).
int synth_normal_quantized(int dtype, uint64_t seed, int64_t rows, int64_t cols, float stdv, uint8_t *out) {
    int64_t rb = row_bytes(dtype, cols);
    if (rb < 0) return 0;
#pragma omp parallel
    {
        std::vector<float> buf((size_t)cols);
#pragma omp for schedule(dynamic, 16)
        for (int64_t r = 0; r < rows; r++) {
            normal_row(seed, (uint64_t)r, stdv, 0.0f, buf.data(), cols);
            quant_row(dtype, buf.data(), cols, out + r * rb);
        }
    }
    return 1;
}

// Uniform token ids in [0, vocab).
void synth_token_ids(uint64_t seed, int64_t n, uint32_t vocab, uint32_t *out) {
    Xoshiro g(seed, 0xABCDEFull);
    for (int64_t i = 0; i < n; i++) out[i] = (uint32_t)(g.next() % vocab);
}

}  // extern "C"

extern "C" {
// RoPE inverse frequencies as build_rope_inv_freq_with_factors computes them
// (src/model.rs:3035-3057, no per-pair factors): 1 / (scaling * theta^(2i/hd)),
// with libm powf on f32 arguments, so the values match the reference's.
void synth_rope_inv_freq(float theta, int64_t head_dim, float scaling, float *out) {
    for (int64_t pair = 0; pair < head_dim / 2; pair++) {
        float i = (float)(pair * 2);
        float base = powf(theta, i / (float)head_dim);
        out[pair] = 1.0f / (scaling * base * 1.0f);
    }
}

// gpt-oss YaRN table as the reference's loader builds it
// (build_rope_inv_freq_gpt_oss, src/model.rs:3059-3098): pairs below `low`
// keep 1/base, pairs above `high` get 1/(scaling*base), a linear ramp in
// between; concentration = 0.1 ln(scaling) + 1.  f32 arithmetic with libm
// logf/powf (Rust's f32::ln / powf), nothing contracted.
void synth_rope_inv_freq_gpt_oss(float theta, int64_t head_dim, float scaling, int64_t orig_ctx, float *out,
                                 float *concentration) {
    const bool yarn = scaling > 1.0f;
    const float two_pi = 2.0f * 3.14159265358979323846f;
    const float half = (float)head_dim / 2.0f;
    // 32 and 1 are the fast/slow rotation counts of the ramp's ends
    const float lo = yarn ? half * (logf((float)orig_ctx / (32.0f * two_pi)) / logf(theta)) : 0.0f;
    const float hi = yarn ? half * (logf((float)orig_ctx / two_pi) / logf(theta)) : 0.0f;
    *concentration = yarn ? 0.1f * logf(scaling) + 1.0f : 1.0f;
    for (int64_t pair = 0; pair < head_dim / 2; pair++) {
        const float base = powf(theta, (float)(2 * pair) / (float)head_dim);
        if (!yarn) {
            out[pair] = 1.0f / base;
            continue;
        }
        float r = ((float)pair - lo) / (hi - lo);
        r = std::min(1.0f, std::max(0.0f, r));
        const float keep = 1.0f - r;  // weight of the extrapolated frequency
        out[pair] = (1.0f / (scaling * base)) * (1.0f - keep) + (1.0f / base) * keep;
    }
}
}
