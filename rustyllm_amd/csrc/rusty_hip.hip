// rusty_hip.hip — host side of librusty_hip.so: device context, weight cache,
// kernel launch helpers, the C ABI declared in include/rusty_hip.h and the
// resident (whole-token-on-device) decoder.
//
// One translation unit: the kernel sources are included so launches see the
// templates directly.
#include "gemv.hip"
#include "attention.hip"
#include "ops.hip"
#include "attention_exact.hip"
#include "moe.hip"
#include "gemm_mfma.hip"
#include "prefill.hip"
#include "prefill_moe.hip"
#include "gguf.hpp"

#include <hip/hip_ext.h>

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/rusty_hip.h"

// Device scratch of rusty_hip_attention_noalloc: the exact-attention scores,
// coefficients and masks, or the split-K partials, of one call.  Every GPU
// holds its own copy for the life of the process; host code uses the address
// hipGetSymbolAddress returns for the current device (Ctx::noalloc), never
// this name, which on the host is only a stand-in.
#define RH_NOALLOC_SCRATCH_BYTES (16u << 20)
static __device__ __align__(256) float scratch[RH_NOALLOC_SCRATCH_BYTES / 4];

namespace rh {

// ---- errors -------------------------------------------------------------------
static bool debug_on() {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("RUSTY_HIP_DEBUG");
        v = (e && *e && strcmp(e, "0") != 0) ? 1 : 0;
    }
    return v == 1;
}
#define RH_CHECK(expr)                                                                          \
    do {                                                                                        \
        hipError_t _e = (expr);                                                                 \
        if (_e != hipSuccess) {                                                                 \
            if (debug_on()) fprintf(stderr, "[rusty_hip] %s failed: %s (%s:%d)\n", #expr,       \
                                    hipGetErrorString(_e), __FILE__, __LINE__);                 \
            return 0;                                                                           \
        }                                                                                       \
    } while (0)
#define RH_LAUNCH_OK()                                                                          \
    do {                                                                                        \
        hipError_t _e = hipGetLastError();                                                      \
        if (_e != hipSuccess) {                                                                 \
            if (debug_on()) fprintf(stderr, "[rusty_hip] launch failed: %s (%s:%d)\n",          \
                                    hipGetErrorString(_e), __FILE__, __LINE__);                 \
            return 0;                                                                           \
        }                                                                                       \
    } while (0)

// ---- context --------------------------------------------------------------------
struct DevW {
    const uint8_t *p = nullptr;
    int64_t stride = 0;
    int32_t rows = 0, cols = 0, fmt = 0;
    uint64_t fp = 0;  // sampled fingerprint of the host bytes it was copied from
};

struct KeyHash {
    size_t operator()(const std::pair<const void *, size_t> &k) const {
        return std::hash<const void *>()(k.first) ^ (std::hash<size_t>()(k.second) * 0x9E3779B97F4A7C15ull);
    }
};

struct Profile {
    std::map<std::string, int> index;
    std::vector<std::string> names;
    std::vector<double> total_ms;
    std::vector<int64_t> count;
    std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> pending;
    std::vector<hipEvent_t> pool;
    bool on = false;
    struct ProfScope *cur = nullptr;  // scope whose launches rh_launch times
};

struct Ctx {
    int state = 0;  // 0 = untried, 1 = ok, -1 = failed
    int dev = 0;
    int n_cu = 256;
    hipStream_t s = nullptr;
    std::mutex mu;
    std::unordered_map<std::pair<const void *, size_t>, DevW, KeyHash> wcache;
    // per-op staging
    float *x = nullptr, *y = nullptr, *y2 = nullptr, *y3 = nullptr, *hid = nullptr, *hid2 = nullptr;
    size_t x_cap = 0, y_cap = 0, hid_cap = 0;
    XQ xq{};
    size_t xq_cap = 0;
    XQ xq2{};
    size_t xq2_cap = 0;
    float *part = nullptr;
    size_t part_cap = 0;
    float *moe = nullptr;  // MoE block scratch: logits, probs, gate, up, proj (+ int32 selection)
    size_t moe_cap = 0;
    float *kv_k = nullptr, *kv_v = nullptr;
    size_t kv_cap = 0;
    int32_t *ibuf = nullptr;
    size_t ibuf_cap = 0;
    float *ex = nullptr;  // exact-attention scratch: scores | coef | masks
    size_t ex_cap = 0;
    int8_t *bq = nullptr;  // batched Q8_K activations: quants [T][K] | scales [K/256][ldx]
    size_t bq_cap = 0;
    float *bx = nullptr, *by = nullptr;  // batched inputs / outputs of the per-op batch export
    size_t bx_cap = 0, by_cap = 0;
    int attn_fast = -1;   // -1: read RUSTY_HIP_ATTN once; 0 exact, 1 split-K
    Profile prof;
    float *noalloc[16] = {};  // device address of `scratch`, per device (set up by init)
    uint8_t *stage[2] = {nullptr, nullptr};  // pinned staging of weight uploads
    hipEvent_t stage_ev[2] = {nullptr, nullptr};
};
static Ctx g;

static int64_t row_bytes_of(int fmt, int64_t cols) {
    switch (fmt) {
    case 0: return cols * 4;
    case 8: return (cols / 32) * 34;
    case 12: return (cols / 256) * 144;
    case 14: return (cols / 256) * 210;
    case 39: return (cols / 32) * 17;
    default: return -1;
    }
}
static int block_elems(int fmt) { return (fmt == 12 || fmt == 14) ? 256 : (fmt == 0 ? 1 : 32); }

static int init_locked() {
    if (g.state != 0) return g.state == 1;
    g.state = -1;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    RH_CHECK(hipSetDevice(0));
    hipDeviceProp_t prop;
    RH_CHECK(hipGetDeviceProperties(&prop, 0));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        if (debug_on()) fprintf(stderr, "[rusty_hip] device is %s, built for gfx950\n", prop.gcnArchName);
        return 0;
    }
    g.n_cu = prop.multiProcessorCount;
    RH_CHECK(hipStreamCreateWithFlags(&g.s, hipStreamNonBlocking));
    // the no-allocation entry point's scratch on this device (device 0 is current)
    void *sp = nullptr;
    if (hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)) != hipSuccess || !sp) {
        if (debug_on()) fprintf(stderr, "[rusty_hip] no address for the no-allocation scratch\n");
        sp = nullptr;
    }
    g.noalloc[g.dev] = (float *)sp;
    g.state = 1;
    return 1;
}

template <class T>
static int ensure(T **p, size_t *cap, size_t n) {
    if (*cap >= n && *p) return 1;
    if (*p) RH_CHECK(hipFree(*p));
    *p = nullptr;
    size_t want = n < 256 ? 256 : n;
    RH_CHECK(hipMalloc((void **)p, want * sizeof(T)));
    *cap = want;
    return 1;
}

static int alloc_xq(XQ *xq, size_t n) {
    size_t nb = (n + 255) / 256;
    RH_CHECK(hipMalloc((void **)&xq->qs, nb * 256));
    RH_CHECK(hipMalloc((void **)&xq->d, nb * sizeof(float)));
    RH_CHECK(hipMalloc((void **)&xq->bsums, nb * 8 * sizeof(int16_t)));
    RH_CHECK(hipMalloc((void **)&xq->sums16, nb * 16 * sizeof(int16_t)));
    return 1;
}
static void free_xq(XQ *xq) {
    if (xq->qs) (void)hipFree(xq->qs);
    if (xq->d) (void)hipFree(xq->d);
    if (xq->bsums) (void)hipFree(xq->bsums);
    if (xq->sums16) (void)hipFree(xq->sums16);
    *xq = XQ{};
}
static int ensure_xq(XQ *xq, size_t *cap, size_t n) {
    if (*cap >= n && xq->qs) return 1;
    free_xq(xq);
    if (!alloc_xq(xq, n)) return 0;
    *cap = (n + 255) / 256 * 256;
    return 1;
}

// FNV-1a over 256 16-byte samples spread across the buffer (plus both
// ends): cheap next to an upload, and it catches a host address that was
// freed and reused for different bytes.
static uint64_t fingerprint(const uint8_t *p, size_t len) {
    uint64_t h = 1469598103934665603ull ^ len;
    auto mix = [&](size_t off) {
        size_t n = std::min<size_t>(16, len - off);
        for (size_t i = 0; i < n; i++) h = (h ^ p[off + i]) * 1099511628211ull;
    };
    if (len == 0) return h;
    for (int k = 0; k < 256; k++) mix((size_t)((unsigned __int128)len * k / 256));
    mix(len > 16 ? len - 16 : 0);
    return h;
}

static bool weight_shape_ok(const uint8_t *host, size_t len, int64_t rows, int64_t cols, int fmt) {
    if (!host || rows <= 0 || cols <= 0) return false;
    int64_t rb = row_bytes_of(fmt, cols);
    if (rb <= 0 || cols % block_elems(fmt) != 0) return false;
    return (int64_t)len >= rows * rb;
}

// rows x rb host bytes (pageable, e.g. a mapped file) into device rows of
// `stride` bytes through two pinned buffers: while the DMA of one chunk runs,
// the host copies (and pages in) the next.  Synchronous.
#define RH_STAGE_BYTES ((size_t)32 << 20)
static hipError_t staged_upload(uint8_t *d, int64_t stride, const uint8_t *host, int64_t rb, int64_t rows) {
    if (!g.stage[0]) {
        for (int i = 0; i < 2; i++) {
            hipError_t e = hipHostMalloc((void **)&g.stage[i], RH_STAGE_BYTES, hipHostMallocDefault);
            if (e == hipSuccess) e = hipEventCreateWithFlags(&g.stage_ev[i], hipEventDisableTiming);
            if (e != hipSuccess) return e;
        }
    }
    const int64_t per = std::max<int64_t>(1, (int64_t)RH_STAGE_BYTES / rb);
    int i = 0;
    for (int64_t r0 = 0; r0 < rows; r0 += per, i ^= 1) {
        const int64_t n = std::min(per, rows - r0);
        hipError_t e = hipEventSynchronize(g.stage_ev[i]);  // this buffer's previous DMA is done
        if (e != hipSuccess) return e;
        memcpy(g.stage[i], host + r0 * rb, (size_t)(n * rb));
        e = hipMemcpy2DAsync(d + r0 * stride, (size_t)stride, g.stage[i], (size_t)rb, (size_t)rb, (size_t)n,
                             hipMemcpyHostToDevice, g.s);
        if (e == hipSuccess) e = hipEventRecord(g.stage_ev[i], g.s);
        if (e != hipSuccess) return e;
    }
    return hipStreamSynchronize(g.s);
}

// A new device copy of a host weight (the caller owns it).  Rows are padded
// to a 16-byte stride; block bytes are copied unchanged.
static int upload_weight(const uint8_t *host, int64_t rows, int64_t cols, int fmt, uint64_t fp, DevW *out) {
    const int64_t rb = row_bytes_of(fmt, cols);
    const int64_t stride = (rb + 15) / 16 * 16;
    uint8_t *d = nullptr;
    RH_CHECK(hipMalloc((void **)&d, (size_t)(rows * stride)));
    hipError_t e;
    if ((size_t)(rows * rb) >= ((size_t)4 << 20) && (size_t)rb <= RH_STAGE_BYTES)
        e = staged_upload(d, stride, host, rb, rows);
    else
        e = stride == rb ? hipMemcpy(d, host, (size_t)(rows * rb), hipMemcpyHostToDevice)
                         : hipMemcpy2D(d, (size_t)stride, host, (size_t)rb, (size_t)rb, (size_t)rows,
                                       hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        RH_CHECK(e);
    }
    DevW w;
    w.p = d;
    w.stride = stride;
    w.rows = (int32_t)rows;
    w.cols = (int32_t)cols;
    w.fmt = fmt;
    w.fp = fp;
    *out = w;
    return 1;
}

// Device copy of a host weight for the per-op exports, cached by (pointer,
// length) and checked against a sampled fingerprint of the bytes.  The
// resident decoder keeps copies of its own (r_weight), so neither eviction
// here nor rusty_hip_weight_cache_clear can pull memory from under it.
static int get_weight(const uint8_t *host, size_t len, int64_t rows, int64_t cols, int fmt, DevW *out) {
    if (!weight_shape_ok(host, len, rows, cols, fmt)) return 0;
    auto key = std::make_pair((const void *)host, len);
    auto it = g.wcache.find(key);
    uint64_t fp = fingerprint(host, len);
    if (it != g.wcache.end()) {
        if (it->second.rows == rows && it->second.cols == cols && it->second.fmt == fmt && it->second.fp == fp) {
            *out = it->second;
            return 1;
        }
        (void)hipStreamSynchronize(g.s);
        (void)hipFree((void *)it->second.p);
        g.wcache.erase(it);
    }
    DevW w;
    if (!upload_weight(host, rows, cols, fmt, fp, &w)) return 0;
    g.wcache[key] = w;
    *out = w;
    return 1;
}

// Frees every cached device copy.  Needed when host weight memory is freed and
// its addresses may be reused for different bytes (the reference never frees
// its mmap'd weights, so its cache has no such call).
static void wcache_clear() {
    (void)hipStreamSynchronize(g.s);
    for (auto &kv : g.wcache) (void)hipFree((void *)kv.second.p);
    g.wcache.clear();
}

// ---- profiling -------------------------------------------------------------------
// A scope names one launch family.  Its kernel is timed by the dispatch
// itself (hipExtLaunchKernel's start/stop events are stamped from the AQL
// packet's own begin/end), which is the interval a kernel trace reports; a
// scope that issues several launches stops at the end of its last one.
struct ProfScope {
    int idx = -1;
    int launches = 0;
    hipEvent_t a = nullptr, b = nullptr;
    hipStream_t stream = nullptr;
    ProfScope(const char *name, hipStream_t s) {
        if (!g.prof.on) return;
        auto it = g.prof.index.find(name);
        if (it == g.prof.index.end()) {
            idx = (int)g.prof.names.size();
            g.prof.index[name] = idx;
            g.prof.names.push_back(name);
            g.prof.total_ms.push_back(0.0);
            g.prof.count.push_back(0);
        } else {
            idx = it->second;
        }
        a = take();
        b = take();
        if (!a || !b) {
            idx = -1;
            return;
        }
        stream = s;
        g.prof.cur = this;
    }
    ~ProfScope() {
        if (idx < 0) return;
        if (g.prof.cur == this) g.prof.cur = nullptr;
        if (launches == 0) {
            g.prof.pool.push_back(a);
            g.prof.pool.push_back(b);
            return;
        }
        if (launches > 1) (void)hipEventRecord(b, stream);
        g.prof.pending.push_back({idx, {a, b}});
    }
    static hipEvent_t take() {
        if (!g.prof.pool.empty()) {
            hipEvent_t e = g.prof.pool.back();
            g.prof.pool.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        return e;
    }
};

// Every library launch goes through here: inside an active profiling scope
// the first launch carries the scope's events.
template <class F, class... Args>
static void rh_launch(F kernel, dim3 grid, dim3 block, uint32_t shm, hipStream_t s, Args... args) {
    ProfScope *ps = g.prof.cur;
    if (ps && ps->stream == s && ps->launches++ == 0)
        hipExtLaunchKernelGGL(kernel, grid, block, shm, s, ps->a, ps->b, 0u, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, shm, s, args...);
}

static void prof_drain() {
    if (g.prof.pending.empty()) return;
    (void)hipStreamSynchronize(g.s);
    for (auto &p : g.prof.pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.second.first, p.second.second) == hipSuccess) {
            g.prof.total_ms[p.first] += ms;
            g.prof.count[p.first] += 1;
        }
        g.prof.pool.push_back(p.second.first);
        g.prof.pool.push_back(p.second.second);
    }
    g.prof.pending.clear();
}

// ---- launch helpers -------------------------------------------------------------
struct MatSpec {
    DevW w;
    float *y;
    const float *bias;
};

// The activation a GEMV call consumes.  ACT_XQ: xq holds the Q8_K vector and
// x the f32 one.  The other modes name the op that produces it from x
// (quantize, RMSNorm then quantize, attention normalisation then quantize);
// the GEMV call runs that op's kernel into xq (and xn) first.
enum ActMode : int { ACT_XQ = 0, ACT_QUANT = 1, ACT_RMSNORM = 2, ACT_DEN = 3 };
struct ActSpec {
    int mode;
    float *x;
    const float *norm_w;
    float eps;
    const float *den;
    int group;
    XQ xq;
    float *xn;
};
static ActSpec act_xq(const XQ &xq, const float *x) {
    ActSpec a;
    memset(&a, 0, sizeof(a));
    a.mode = ACT_XQ;
    a.xq = xq;
    a.x = (float *)x;
    return a;
}

enum Cat { CAT_KQ = 1, CAT_Q8I = 2, CAT_F32 = 3 };
static int cat_of(int fmt, int K) {
    if (fmt == 12 || fmt == 14) return K % 256 == 0 && K <= KMAX ? CAT_KQ : 0;
    if (fmt == 8) {
        if (K % 256 == 0 && K <= KMAX) return CAT_Q8I;
        return K % 32 == 0 && K <= 12288 ? CAT_F32 : 0;
    }
    if (fmt == 39) return K % 32 == 0 && K <= KMAX ? CAT_F32 : 0;
    return 0;
}

static int grid_cap() { return g.n_cu * 8; }

// Persistent grid: as many workgroups as fit on the device at once (queried
// once per kernel instantiation), never more than the tiles need.
// Kinds of persistent GEMV launch, for the per-CU workgroup cap of launches
// that build their activation in a prologue.
enum GridKind { GK_PLAIN = 0, GK_PRO = 1, GK_PRO_SWIGLU = 2, GK_PRO_SPLIT = 3, GK_PRO_KQ2 = 4 };
template <class Kern>
static int persistent_grid(Kern kernel, int n_tiles, int waves_per_wg, int kind = GK_PLAIN) {
    // RUSTY_HIP_WG_PER_CU caps the resident workgroups per CU (sweeps)
    static std::map<const void *, int> occ;
    auto it = occ.find((const void *)kernel);
    int per_cu;
    if (it == occ.end()) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel, 256, 0) != hipSuccess || nb <= 0) nb = 2;
        occ[(const void *)kernel] = nb;
        per_cu = nb;
    } else {
        per_cu = it->second;
    }
    // Launches that build their activation in a prologue run at most three
    // resident workgroups per CU (two for the two-format q/k/v launch): each wave then takes more tiles through its
    // two-deep load pipeline, which amortises the prologue (8B decode: 2 per
    // CU 342.5, 3 per CU 350.5, 4 per CU 340.7 tok/s); the others keep the
    // occupancy limit, which streams faster on its own (Q4_K 14336x4096: 11.0
    // against 12.6 us).
    // RUSTY_HIP_WG_CAPS="a,b,c,d" sets the prologue caps per kind (plain,
    // SwiGLU, row-split, two-format)
    static int cap = -1;
    static int pcap[5] = {0, 3, 3, 3, 2};  // q/k/v: 351.6 at 2 against 349.7 at 3
    if (cap < 0) {
        const char *e = getenv("RUSTY_HIP_WG_PER_CU");
        cap = e ? atoi(e) : 0;
        const char *c = getenv("RUSTY_HIP_WG_CAPS");
        if (c) sscanf(c, "%d,%d,%d,%d", &pcap[1], &pcap[2], &pcap[3], &pcap[4]);
    }
    if (cap > 0) per_cu = std::min(per_cu, cap);
    else if (kind != GK_PLAIN && pcap[kind] > 0) per_cu = std::min(per_cu, pcap[kind]);
    int need = (n_tiles + waves_per_wg - 1) / waves_per_wg;
    int grid = std::min(need, per_cu * g.n_cu);
    return grid < 1 ? 1 : grid;
}

template <int FMT, bool SW, int U, int ACT>
static int launch_kq_act(const GemvArgs &A, hipStream_t s) {
    auto kern = gemv_kq_kernel<FMT, SW, U, ACT>;
    int grid = persistent_grid(kern, A.n_tiles, 4, ACT == KQ_ACT_XQ ? GK_PLAIN : SW ? GK_PRO_SWIGLU : GK_PRO);
    ProfScope ps(SW ? "gemv_kquant_swiglu" : "gemv_kquant", s);
    rh_launch(kern, dim3(grid), dim3(256), 0, s, A);
    RH_LAUNCH_OK();
    return 1;
}
template <int FMT, int ACT>
static int launch_kq_split_act(const GemvArgs &A, hipStream_t s) {
    auto kern = gemv_kq_kernel<FMT, false, 1, ACT, true>;
    int grid = persistent_grid(kern, A.n_tiles * 4, 4, ACT == KQ_ACT_XQ ? GK_PLAIN : GK_PRO_SPLIT);  // four waves per tile
    ProfScope ps("gemv_kquant", s);
    rh_launch(kern, dim3(grid), dim3(256), 0, s, A);
    RH_LAUNCH_OK();
    return 1;
}
template <int FMT>
static int launch_kq_split(const GemvArgs &A, int act, hipStream_t s) {
    if (act == KQ_ACT_NORM) return launch_kq_split_act<FMT, KQ_ACT_NORM>(A, s);
    if (act == KQ_ACT_DEN) return launch_kq_split_act<FMT, KQ_ACT_DEN>(A, s);
    if (act == KQ_ACT_QUANT) return launch_kq_split_act<FMT, KQ_ACT_QUANT>(A, s);
    return launch_kq_split_act<FMT, KQ_ACT_XQ>(A, s);
}
template <int FMT, bool SW, int U>
static int launch_kq(const GemvArgs &A, int act, hipStream_t s) {
    if (act == KQ_ACT_NORM) return launch_kq_act<FMT, SW, U, KQ_ACT_NORM>(A, s);
    if (act == KQ_ACT_DEN) return launch_kq_act<FMT, SW, U, KQ_ACT_DEN>(A, s);
    if (act == KQ_ACT_NORM2) return launch_kq_act<FMT, SW, U, KQ_ACT_NORM2>(A, s);
    if (act == KQ_ACT_DEN2) {
        if constexpr (SW || U > 2) return 0;  // (wo: one row of fewer than 32 blocks in two units)
        else return launch_kq_act<FMT, SW, U, KQ_ACT_DEN2>(A, s);
    }
    if (act == KQ_ACT_QUANT) return launch_kq_act<FMT, SW, U, KQ_ACT_QUANT>(A, s);
    return launch_kq_act<FMT, SW, U, KQ_ACT_XQ>(A, s);
}
template <int W, int ACT, bool SW>
static int launch_q8p(const GemvArgs &A, hipStream_t s) {
    // one workgroup per CU (the wave-private transposes take most of the LDS)
    const int grid = std::max(1, std::min((A.n_tiles + W - 1) / W, g.n_cu));
    ProfScope ps("gemv_q8_0_int", s);
    rh_launch((gemv_q8_0_pipe_kernel<W, ACT, SW>), dim3(grid), dim3(64 * W), 0, s, A);
    RH_LAUNCH_OK();
    return 1;
}
template <int W>
static int launch_q8p_w(const GemvArgs &A, int act, bool sw, hipStream_t s) {
    if (sw) return act == KQ_ACT_NORM ? launch_q8p<W, KQ_ACT_NORM, true>(A, s) : launch_q8p<W, KQ_ACT_XQ, true>(A, s);
    switch (act) {
    case KQ_ACT_NORM: return launch_q8p<W, KQ_ACT_NORM, false>(A, s);
    case KQ_ACT_DEN: return launch_q8p<W, KQ_ACT_DEN, false>(A, s);
    case KQ_ACT_QUANT: return launch_q8p<W, KQ_ACT_QUANT, false>(A, s);
    default: return launch_q8p<W, KQ_ACT_XQ, false>(A, s);
    }
}
// Waves per workgroup W: the fewest tiles on the busiest CU,
// W * ceil(tiles / (W * CUs)), ties to the larger W (more loads in flight);
// RUSTY_HIP_Q8P_WAVES=1/2/4/7 forces one (sweeps).
static int launch_q8p_any(const GemvArgs &A, int act, bool sw, hipStream_t s) {
    if (sw && act != KQ_ACT_NORM && act != KQ_ACT_XQ) return 0;
    static int forced = -1;
    if (forced < 0) {
        const char *e = getenv("RUSTY_HIP_Q8P_WAVES");
        forced = e ? atoi(e) : 0;
    }
    int w = forced;
    if (w != 1 && w != 2 && w != 4 && w != 7) {
        const int cands[4] = {1, 2, 4, 7};
        long best = -1;
        for (int c : cands) {
            const long f = (long)c * ((A.n_tiles + (long)c * g.n_cu - 1) / ((long)c * g.n_cu));
            if (best < 0 || f <= best) best = f, w = c;
        }
    }
    switch (w) {
    case 1: return launch_q8p_w<1>(A, act, sw, s);
    case 2: return launch_q8p_w<2>(A, act, sw, s);
    case 4: return launch_q8p_w<4>(A, act, sw, s);
    default: return launch_q8p_w<7>(A, act, sw, s);
    }
}
// RUSTY_HIP_MX_SERIAL_PER_CU: tiles per CU up to which the producer/adder
// workgroups serve an MXFP4 launch (two per CU fit in LDS, but measured
// slower on the gpt-oss expert launches: 279 against 285 tok/s)
// LDS bytes of the fused MXFP4 kernel's x (K floats rounded up to 256), and
// the largest K it serves: with its 17 KB chunk, at most 64 KB per workgroup
static size_t mx_fused_x_bytes(int K) { return (size_t)(K + 255) / 256 * 1024; }
static bool mx_fused_fits(int K) { return 17408 + mx_fused_x_bytes(K) <= 65536; }
static int mx_serial_per_cu() {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("RUSTY_HIP_MX_SERIAL_PER_CU");
        v = e ? atoi(e) : 1;
    }
    return v;
}
template <int FMT>
static int launch_f32x(const GemvArgs &A, hipStream_t s) {
    if constexpr (FMT == F_MXFP4) {
        ProfScope ps("gemv_mxfp4", s);
        if (A.n_tiles > mx_serial_per_cu() * g.n_cu && mx_fused_fits(A.K)) {
            // more tiles than CUs: one wave per tile computes its own terms,
            // several tiles per SIMD
            rh_launch(gemv_mxfp4_fused_kernel<false>, dim3(A.n_tiles), dim3(64), mx_fused_x_bytes(A.K), s, A);
        } else {
            // one workgroup per tile: the serial row sums are spread over a
            // summing wave and MXP term-producing waves
            rh_launch(gemv_mxfp4_serial_kernel<MXP>, dim3(A.n_tiles), dim3(64 * (MXP + 1)), 0, s, A);
        }
        RH_LAUNCH_OK();
        return 1;
    } else {
        static_assert(FMT == F_Q8_0, "f32-activation formats: Q8_0 and MXFP4");
        // one workgroup per 8-row tile
        ProfScope ps("gemv_f32x", s);
        rh_launch(gemv_q8_0_f32x_kernel<false>, dim3(A.n_tiles), dim3(64), (uint32_t)(A.K * sizeof(float)), s, A);
        RH_LAUNCH_OK();
        return 1;
    }
}
// K-quant tiles: it = units per lane (a wave tile is 64*it quarter-block
// units of r whole rows; SWIGLU tiles hold r gate + r up rows).  The fewest
// units that hold one row (pair): small tiles give each wave more tiles
// through its two-deep load pipeline, which measured faster at every decode
// shape (Q6_K 14336x4096 cold: 18.2 us at 4 units, 13.5 at 1; 128256x4096
// unchanged).  RUSTY_HIP_KQ_U forces a preferred value.
static int kq_units_per_lane(int K, int rows, bool swiglu) {
    const int nb = K / 256;
    const int need = ((swiglu ? 2 : 1) * nb * 4 + 63) / 64;  // one row (pair) must fit
    static int forced = -1;
    if (forced < 0) {
        const char *e = getenv("RUSTY_HIP_KQ_U");
        forced = e ? atoi(e) : 0;
    }
    (void)rows;
    const int pref = forced > 0 ? forced : 1;
    int u = std::max(pref, need);
    return u > 4 ? 0 : u;
}
// Rows per wave tile: all units fit the wave (4*rows*nb <= 64*U quarter
// blocks) and the block values fit its LDS row buffer (rows padded to a
// multiple of 4 blocks, 64 slots).
static int kq_tile_rows(int K, int units_per_lane, bool swiglu) {
    const int nb = K / 256, nbp = (nb + 3) & ~3, m = swiglu ? 2 : 1;
    return std::max(1, std::min(16 * units_per_lane / nb, 64 / nbp) / m);
}

// rows per wave tile of a category's kernel
static void pick_iters(int cat, int K, int *it, int *r) {
    (void)K;
    // K-quant: one row per wave tile (units per lane chosen by the caller);
    // Q8_0 int: gemv_q8_0_pipe_kernel's 8-row wave tiles
    *it = cat == CAT_Q8I ? 0 : 1;
    *r = cat == CAT_Q8I ? 2 : 1;
}

// The prologue mode a K-quant launch uses to build act itself, or -1 when a
// standalone kernel has to produce the Q8_K vector first.
static int kq_prologue_act(const ActSpec &a, int K) {
    static int off = -1;
    if (off < 0) {
        const char *e = getenv("RUSTY_HIP_ACT_PROLOGUE");  // 0: always the standalone kernels
        off = (e && atoi(e) == 0) ? 1 : 0;
    }
    if (a.mode == ACT_XQ) return KQ_ACT_XQ;
    if (off || K % 256 != 0) return -1;
    if (a.mode == ACT_QUANT && K <= KQ_ACT_QUANT_KMAX && ((uintptr_t)a.x & 15) == 0) return KQ_ACT_QUANT;
    if (K > KQ_ACT_KMAX2) return -1;
    const bool wide = K > KQ_ACT_KMAX;  // two 16-element chunks per thread
    if (a.mode == ACT_RMSNORM && ((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.norm_w & 15) == 0)
        return wide ? KQ_ACT_NORM2 : KQ_ACT_NORM;
    if (a.mode == ACT_DEN && a.group > 0 && a.group % 16 == 0 && ((uintptr_t)a.x & 15) == 0)
        return wide ? KQ_ACT_DEN2 : KQ_ACT_DEN;
    return -1;
}
// The prologues the Q8_0 integer kernel builds: those of K-quant up to
// K = 4096 (NORM stages K + 128 floats in its staging of KQ_XQ_WORDS).
static int q8_prologue_act(const ActSpec &a, int K) {
    const int k = kq_prologue_act(a, K);
    return (k == KQ_ACT_NORM2 || k == KQ_ACT_DEN2) ? -1 : k;
}

// The launch arguments for y_i = W_i x over matrices of one category: the
// category, units per lane (it) and activation mode (kact) of the launch.
// Row-split K-quant tiles (KQ_SPLIT): plain rows of at least 32 blocks are
// shared by a workgroup's four waves, one unit per lane.
static bool kq_split(int K, int epi) {
    static int off = -1;
    if (off < 0) {
        const char *e = getenv("RUSTY_HIP_KQ_SPLIT");  // 0: rows of one wave
        off = (e && atoi(e) == 0) ? 1 : 0;
    }
    return !off && epi != EPI_SWIGLU && K / 256 >= 32;
}

static int gemv_cat_args(const MatSpec *ms, int n, int K, int epi, const ActSpec &act, GemvArgs &A, int &cat_out,
                         int &it_out, int &kact_out) {
    if (n <= 0 || n > GEMV_MAX_MATS) return 0;
    int cat = cat_of(ms[0].w.fmt, K);
    if (!cat) return 0;
    for (int i = 1; i < n; i++)
        if (cat_of(ms[i].w.fmt, K) != cat) return 0;
    int it, r;
    pick_iters(cat, K, &it, &r);
    if (cat == CAT_KQ) {
        int rows = 0;
        for (int i = 0; i < n; i++) rows += ms[i].w.rows;
        it = kq_units_per_lane(K, rows, epi == EPI_SWIGLU);
        r = kq_tile_rows(K, it, epi == EPI_SWIGLU);
        if (kq_split(K, epi)) it = 1, r = 1;  // one row per workgroup tile
    }
    const int kact = cat == CAT_KQ ? kq_prologue_act(act, K)
                     : cat == CAT_Q8I ? q8_prologue_act(act, K)
                                      : (act.mode == ACT_XQ ? KQ_ACT_XQ : -1);
    if (kact < 0) return 0;
    memset(&A, 0, sizeof(A));
    A.K = K;
    A.epi = epi;
    A.xq = act.xq;
    A.x = act.x;
    A.n_mats = n;
    A.act_x = act.x;
    A.act_w = act.norm_w;
    A.act_den = act.den;
    A.act_eps = act.eps;
    A.act_group = act.group;
    A.act_store = (kact > 0 && act.xq.qs) ? 1 : 0;
    int tiles = 0;
    int rows_per_tile = (cat == CAT_KQ) ? r : (cat == CAT_F32) ? (ms[0].w.fmt == 8 ? 8 : 64) : 4 * r;
    if (cat == CAT_Q8I && epi == EPI_SWIGLU) rows_per_tile = 4;  // 4 gate + the same 4 up rows per wave tile
    if (cat == CAT_F32)
        for (int i = 1; i < n; i++)
            if (ms[i].w.fmt != ms[0].w.fmt) return 0;  // one format per launch
    for (int i = 0; i < n; i++) {
        GemvMat &m = A.m[i];
        m.w = ms[i].w.p;
        m.row_stride = ms[i].w.stride;
        m.rows = ms[i].w.rows;
        m.fmt = ms[i].w.fmt;
        m.y = ms[i].y;
        m.bias = ms[i].bias;
        m.tile_begin = (epi == EPI_SWIGLU) ? 0 : tiles;
        if (epi != EPI_SWIGLU) tiles += (m.rows + rows_per_tile - 1) / rows_per_tile;
    }
    if (epi == EPI_SWIGLU) {
        if (n != 2 || (cat != CAT_KQ && cat != CAT_Q8I) || A.m[0].rows != A.m[1].rows ||
            A.m[0].row_stride != A.m[1].row_stride || ms[0].bias || ms[1].bias)
            return 0;
        tiles = (A.m[0].rows + rows_per_tile - 1) / rows_per_tile;
    }
    A.n_tiles = tiles;
    A.tile_rows = r;
    if (cat == CAT_KQ)
        for (int i = 1; i < n; i++)  // gemv_multi groups by format; the kernel assumes one row stride
            if (A.m[i].fmt != A.m[0].fmt || A.m[i].row_stride != A.m[0].row_stride) return 0;
    cat_out = cat;
    it_out = it;
    kact_out = kact;
    return 1;
}

// Launches y_i = W_i x for matrices of one category.
static int gemv_cat(const MatSpec *ms, int n, int K, int epi, const ActSpec &act, hipStream_t s) {
    GemvArgs A;
    int cat, it, kact;
    if (!gemv_cat_args(ms, n, K, epi, act, A, cat, it, kact)) return 0;
    if (cat == CAT_KQ && kq_split(K, epi))
        return A.m[0].fmt == 12 ? launch_kq_split<F_Q4_K>(A, kact, s) : launch_kq_split<F_Q6_K>(A, kact, s);
    if (cat == CAT_KQ) {
        const bool q4 = A.m[0].fmt == 12;
#define RH_KQ_U(U)                                                                                     \
    if (it == U) {                                                                                     \
        if (epi == EPI_SWIGLU)                                                                         \
            return q4 ? launch_kq<F_Q4_K, true, U>(A, kact, s) : launch_kq<F_Q6_K, true, U>(A, kact, s); \
        return q4 ? launch_kq<F_Q4_K, false, U>(A, kact, s) : launch_kq<F_Q6_K, false, U>(A, kact, s);   \
    }
        RH_KQ_U(1) RH_KQ_U(2) RH_KQ_U(3) RH_KQ_U(4)
#undef RH_KQ_U
        return 0;
    }
    if (cat == CAT_Q8I) return launch_q8p_any(A, kact, epi == EPI_SWIGLU, s);
    return A.m[0].fmt == 8 ? launch_f32x<F_Q8_0>(A, s) : launch_f32x<F_MXFP4>(A, s);
}

static int launch_quant(const float *x, int n, const XQ &xq, hipStream_t s);
static int launch_rmsnorm(const float *x, const float *w, float eps, int n, float *xn, const XQ *xq, hipStream_t s);

// Runs the standalone kernel that produces an ActSpec's Q8_K (and f32)
// vector, for launches that cannot build it in their prologue.
static int act_materialize(const ActSpec &a, int K, ActSpec *out, hipStream_t s) {
    switch (a.mode) {
    case ACT_XQ:
        *out = a;
        return 1;
    case ACT_QUANT:
        if (K % 256 == 0 && !launch_quant(a.x, K, a.xq, s)) return 0;
        *out = act_xq(K % 256 == 0 ? a.xq : XQ{}, a.x);
        return 1;
    case ACT_RMSNORM:
        if (!a.xn) return 0;
        if (!launch_rmsnorm(a.x, a.norm_w, a.eps, K, a.xn, K % 256 == 0 ? &a.xq : nullptr, s)) return 0;
        *out = act_xq(K % 256 == 0 ? a.xq : XQ{}, a.xn);
        return 1;
    case ACT_DEN: {
        ProfScope ps("attn_exact_finish", s);
        XQ q = K % 256 == 0 ? a.xq : XQ{};
        rh_launch(attn_exact_finish_kernel, dim3((K + 255) / 256), dim3(256), 0, s, a.x, a.den, a.group, K, q);
        RH_LAUNCH_OK();
        *out = act_xq(q, a.x);
        return 1;
    }
    }
    return 0;
}

// Two K-quant launch groups of different formats (a Q4_K group and a Q6_K
// group) that both build act in their prologue, as one launch: the
// persistent grid is split between them in proportion to their weight bytes.
// Returns 0 (nothing launched) for combinations without an instantiation.
template <int UA, int UB>
static int launch_kq2(const GemvArgs &A, const GemvArgs &B, int bytes_a, int bytes_b, hipStream_t s) {
    auto kern = gemv_kq2_kernel<F_Q4_K, UA, F_Q6_K, UB, KQ_ACT_NORM>;
    const int need_a = (A.n_tiles + 3) / 4, need_b = (B.n_tiles + 3) / 4;
    const int total = persistent_grid(kern, A.n_tiles + B.n_tiles, 4, GK_PRO_KQ2);
    int grid_a = (int)((double)total * bytes_a / ((double)bytes_a + bytes_b) + 0.5);
    grid_a = std::max(1, std::min(grid_a, std::min(need_a, total - 1)));
    const int grid_b = std::max(1, std::min(total - grid_a, need_b));
    ProfScope ps("gemv_kquant", s);
    rh_launch(kern, dim3(grid_a + grid_b), dim3(256), 0, s, A, B, grid_a);
    RH_LAUNCH_OK();
    return 1;
}
static int gemv_kq2(const MatSpec *ga, int na, const MatSpec *gb, int nb, int K, const ActSpec &act, hipStream_t s) {
    static int off = -1;
    if (off < 0) {
        const char *e = getenv("RUSTY_HIP_KQ2");  // 0: one launch per format group
        off = (e && atoi(e) == 0) ? 1 : 0;
    }
    if (off) return 0;
    if (ga[0].w.fmt == 14) std::swap(ga, gb), std::swap(na, nb);
    if (ga[0].w.fmt != 12 || gb[0].w.fmt != 14 || kq_split(K, EPI_STORE)) return 0;
    GemvArgs A, B;
    int ca, ia, ka, cb, ib, kb;
    if (!gemv_cat_args(ga, na, K, EPI_STORE, act, A, ca, ia, ka)) return 0;
    if (!gemv_cat_args(gb, nb, K, EPI_STORE, act, B, cb, ib, kb)) return 0;
    if (ca != CAT_KQ || cb != CAT_KQ || ka != KQ_ACT_NORM || kb != KQ_ACT_NORM) return 0;
    B.act_store = 0;  // A's first workgroup publishes the vector
    long long bytes_a = 0, bytes_b = 0;
    for (int i = 0; i < na; i++) bytes_a += (long long)ga[i].w.rows * ga[i].w.stride;
    for (int i = 0; i < nb; i++) bytes_b += (long long)gb[i].w.rows * gb[i].w.stride;
    const int ba = (int)(bytes_a >> 10), bb = (int)(bytes_b >> 10);
    if (ia == 1 && ib == 1) return launch_kq2<1, 1>(A, B, ba, bb, s);
    if (ia == 2 && ib == 1) return launch_kq2<2, 1>(A, B, ba, bb, s);
    if (ia == 1 && ib == 2) return launch_kq2<1, 2>(A, B, ba, bb, s);
    if (ia == 2 && ib == 2) return launch_kq2<2, 2>(A, B, ba, bb, s);
    return 0;
}

// Splits a list of matrices into launch groups (one per category; K-quant
// groups also share one format) and launches each.
static int gemv_multi_act(const MatSpec *ms, int n, int K, int epi, const ActSpec &act, hipStream_t s) {
    // every launch group K-quant and the prologue able to build act: no
    // standalone activation kernel
    bool prologue = kq_prologue_act(act, K) > 0;
    for (int i = 0; i < n && prologue; i++) prologue = cat_of(ms[i].w.fmt, K) == CAT_KQ;
    if (q8_prologue_act(act, K) > 0 && !prologue) {
        // Q8_0 matrices build the same activation in their prologue (one
        // launch group: all Q8_0)
        prologue = true;
        for (int i = 0; i < n && prologue; i++) prologue = cat_of(ms[i].w.fmt, K) == CAT_Q8I;
    }
    ActSpec use = act;
    if (!prologue && !act_materialize(act, K, &use, s)) return 0;
    // with a prologue, the first launch group publishes the Q8_K vector it
    // builds (act.xq) and later groups read it instead of building it again
    const bool share = prologue && act.xq.qs != nullptr;
    ActSpec later = act_xq(act.xq, act.x);
    int done[GEMV_MAX_MATS] = {0};
    MatSpec grp[GEMV_MAX_MATS][GEMV_MAX_MATS];
    int ngrp[GEMV_MAX_MATS], n_groups = 0;
    for (int i = 0; i < n; i++) {
        if (done[i]) continue;
        int cat = cat_of(ms[i].w.fmt, K);
        if (!cat) return 0;
        int ng = 0;
        for (int j = i; j < n; j++)
            if (!done[j] && cat_of(ms[j].w.fmt, K) == cat && (cat == CAT_Q8I || ms[j].w.fmt == ms[i].w.fmt)) {
                grp[n_groups][ng++] = ms[j];
                done[j] = 1;
            }
        ngrp[n_groups++] = ng;
    }
    // two K-quant groups sharing a prologue: one launch when the pair has an
    // instantiation
    if (n_groups == 2 && prologue && epi == EPI_STORE && gemv_kq2(grp[0], ngrp[0], grp[1], ngrp[1], K, use, s))
        return 1;
    for (int g = 0; g < n_groups; g++)
        if (!gemv_cat(grp[g], ngrp[g], K, epi, (share && g > 0) ? later : use, s)) return 0;
    return 1;
}

static int gemv_multi(const MatSpec *ms, int n, int K, int epi, const XQ &xq, const float *xf, hipStream_t s) {
    return gemv_multi_act(ms, n, K, epi, act_xq(xq, xf), s);
}

static int launch_quant(const float *x, int n, const XQ &xq, hipStream_t s) {
    if (n % 256 != 0) return 0;
    ProfScope ps("quantize_q8k", s);
    rh_launch(quantize_q8k_kernel, dim3(n / 256), dim3(256), 0, s, x, n, xq);
    RH_LAUNCH_OK();
    return 1;
}

static int launch_rmsnorm(const float *x, const float *w, float eps, int n, float *xn, const XQ *xq, hipStream_t s) {
    if (n > 16384 || ((uintptr_t)x & 15)) return 0;
    XQ q = xq ? *xq : XQ{};
    if (xq && n % 256 != 0) q = XQ{};
    ProfScope ps("rmsnorm_q8k", s);
    rh_launch(rmsnorm_q8k_kernel, dim3((n + 255) / 256), dim3(256), (size_t)n * sizeof(float), s, x, w, eps,
                       n, xn, q);
    RH_LAUNCH_OK();
    return 1;
}

__global__ void silu_mul_kernel(const float *g_, const float *u, int n, float *out) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        out[i] = silu_mul_ref(g_[i], u[i]);
}
static int launch_silu(const float *g_, const float *u, int n, float *out, hipStream_t s) {
    ProfScope ps("silu_mul", s);
    rh_launch(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, s, g_, u, n, out);
    RH_LAUNCH_OK();
    return 1;
}

// d = W_gate, W_up -> hidden = silu(gate x) * (up x); K-quant pairs use the
// fused epilogue, other formats two GEMVs plus the SiLU kernel.
static int gemv_swiglu_act(const DevW &gate, const DevW &up, int K, const ActSpec &act, float *hidden,
                           float *tmp_g, float *tmp_u, hipStream_t s) {
    const int gc = cat_of(gate.fmt, K);
    if ((gc == CAT_KQ || gc == CAT_Q8I) && gate.fmt == up.fmt && gate.rows == up.rows && gate.stride == up.stride &&
        (gc == CAT_Q8I || K / 256 <= 32)) {
        MatSpec ms[2] = {{gate, hidden, nullptr}, {up, hidden, nullptr}};
        ActSpec use = act;
        if ((gc == CAT_Q8I ? q8_prologue_act(act, K) : kq_prologue_act(act, K)) < 0 &&
            !act_materialize(act, K, &use, s))
            return 0;
        return gemv_cat(ms, 2, K, EPI_SWIGLU, use, s);
    }
    MatSpec ms[2] = {{gate, tmp_g, nullptr}, {up, tmp_u, nullptr}};
    if (!gemv_multi_act(ms, 2, K, EPI_STORE, act, s)) return 0;
    return launch_silu(tmp_g, tmp_u, gate.rows, hidden, s);
}
static int gemv_swiglu(const DevW &gate, const DevW &up, int K, const XQ &xq, const float *xf, float *hidden,
                       float *tmp_g, float *tmp_u, hipStream_t s) {
    return gemv_swiglu_act(gate, up, K, act_xq(xq, xf), hidden, tmp_g, tmp_u, s);
}

static int attn_launch(const AttnArgs &A, hipStream_t s) {
    dim3 grid(A.n_chunks, A.n_kv);
    {
        ProfScope ps("attn_partial", s);
#define RH_ATT(HD, KM)                                                                            \
    if (A.hd == HD && A.vd == HD && A.kv_mul == KM) {                                            \
        rh_launch((attn_partial_kernel<HD, KM>), grid, dim3(256), 0, s, A);              \
        goto launched;                                                                            \
    }
        RH_ATT(128, 1) RH_ATT(128, 2) RH_ATT(128, 4) RH_ATT(128, 5) RH_ATT(128, 6) RH_ATT(128, 8)
        RH_ATT(64, 1) RH_ATT(64, 2) RH_ATT(64, 4) RH_ATT(64, 5) RH_ATT(64, 6) RH_ATT(64, 8)
#undef RH_ATT
        return 0;
    launched:;
        RH_LAUNCH_OK();
    }
    {
        ProfScope ps("attn_combine", s);
        int total = A.n_heads * A.vd;
        rh_launch(attn_combine_kernel, dim3((total + 255) / 256), dim3(256), 0, s, A);
        RH_LAUNCH_OK();
    }
    return 1;
}
static bool attn_supported(int hd, int vd, int kv_mul) {
    return hd == vd && (hd == 64 || hd == 128) &&
           (kv_mul == 1 || kv_mul == 2 || kv_mul == 4 || kv_mul == 5 || kv_mul == 6 || kv_mul == 8);
}
// Splits per kv head: two workgroups per CU (measured at ctx 32768: 63.6 us
// against 69.5 at four and 71.2 at one), each at least one ATT_TP-position
// sub-tile.  RUSTY_HIP_SPLITK_PER_CU overrides it for sweeps.
static int attn_chunks(int n_kv, int max_ctx) {
    static int per_cu = -1;
    if (per_cu < 0) {
        const char *e = getenv("RUSTY_HIP_SPLITK_PER_CU");
        per_cu = e ? std::max(1, atoi(e)) : 2;
    }
    int want = (per_cu * g.n_cu + n_kv - 1) / n_kv;
    int by_ctx = (max_ctx + ATT_TP - 1) / ATT_TP;
    int c = std::min(want, by_ctx);
    return c < 1 ? 1 : c;
}

// Attention order: 0 = the reference's serial online-softmax order, bit for
// bit (default); 1 = split-K flash decode (within the 1e-4 tolerance, not
// bit-exact).  RUSTY_HIP_ATTN=fast selects 1 before the first call.
static int attn_fast_mode() {
    if (g.attn_fast < 0) {
        const char *e = getenv("RUSTY_HIP_ATTN");
        g.attn_fast = (e && strcmp(e, "fast") == 0) ? 1 : 0;
    }
    return g.attn_fast;
}

static size_t exact_e_floats(int n_kv, int kv_mul, int cap) { return (size_t)n_kv * kv_mul * cap; }

static size_t exact_scratch_floats(int n_kv, int kv_mul, int cap) {
    size_t n = (size_t)n_kv * kv_mul;
    return n * cap + exact_e_floats(n_kv, kv_mul, cap) + n * (cap / 64) + n * (cap / 32) + (n + 63) / 64 * 64;
}

// Launches the exact attention kernels; cap = positions reserved per head
// (multiple of 64, >= the longest range this launch may see).  The output is
// normalised in place and, when xq.qs is set, quantized to Q8_K
// (n_heads * vd must then be a multiple of 256).
// With A.n_tok > 0 the launch covers that many query tokens (grid z), each
// with its own scratch block of exact_scratch_floats; finish must then be
// false (the caller normalises the rows).
// RUSTY_HIP_STREAM=0: the resident decoder's exact attention as separate
// launches instead of the streamed one
static bool stream_enabled() {
    static int on = -1;
    if (on < 0) {
        const char *e = getenv("RUSTY_HIP_STREAM");
        on = (e && e[0] == '0') ? 0 : 1;
    }
    return on == 1;
}

// RUSTY_HIP_CHAIN_TOK4=0: the multi-token recurrence one token per wave
// throughout (the four-token kernel off)
static bool chain_tok4_enabled() {
    static int on = -1;
    if (on < 0) {
        const char *e = getenv("RUSTY_HIP_CHAIN_TOK4");
        on = (e && e[0] == '0') ? 0 : 1;
    }
    return on == 1;
}

// sync: the resident decoder's flag block for the streamed launch (null:
// separate scores, coefficient and chain launches).
static int attn_exact_launch(AttnExactArgs A, float *scratch, const XQ &xq, hipStream_t s, bool finish = true,
                             const float **den_out = nullptr, uint32_t *sync = nullptr) {
    const size_t nh = (size_t)A.n_heads, cap = (size_t)A.cap;
    const int ntl = A.cap / EX_TILE;
    const unsigned nz = A.n_tok > 0 ? (unsigned)A.n_tok : 1u;
    if (A.n_tok > 0) {
        if (finish) return 0;
        A.tok_scratch = (int64_t)exact_scratch_floats(A.n_kv, A.kv_mul, A.cap);
    }
    if (A.lin && (A.n_tok <= 0 || A.vt)) return 0;  // the linear ring view is per token, rows only
    A.scores = scratch;
    A.e = scratch + nh * cap;
    A.tmax = A.e + exact_e_floats(A.n_kv, A.kv_mul, A.cap);
    A.newmask = (uint32_t *)(A.tmax + nh * (cap / 64));
    A.den = (float *)(A.newmask + nh * (cap / 32));
    A.kvec = (A.key_stride % 4 == 0 && A.hd % 4 == 0 && ((uintptr_t)A.k & 15) == 0) ? 1 : 0;
    const int n_out = A.n_heads * A.vd;
    if (xq.qs && n_out % 256 != 0) return 0;
    // the lane-sliced scores kernel: 16-byte K rows, kv_mul <= 8, hd 64 or 128
    const bool s8 = A.kvec && A.kv_mul <= CH_MAXG && (A.hd == 64 || A.hd == 128) && A.slot_count >= EX_TILE;
    if (A.fuse_rope && (!s8 || A.n_tok > 0 || A.rope.hd != A.hd)) {
        // the RoPE + KV store the scores kernel would have done
        ProfScope ps("rope_kv", s);
        const int work = A.rope.n_heads * (A.rope.hd / 2) + A.rope.n_kv * (A.rope.hd / 2) + A.rope.n_kv * A.rope.vd;
        rh_launch(rope_kv_kernel, dim3((work + 255) / 256), dim3(256), 0, s, A.rope);
        RH_LAUNCH_OK();
        A.fuse_rope = 0;
    }
    // the LDS-fed chain kernel needs 16-byte rows of 16-dim slices and a
    // ring that fits the cache (its row offsets are 32-bit); it computes the
    // coefficients itself
    const bool c4 = A.vd % 16 == 0 && A.value_stride % 4 == 0 && ((uintptr_t)A.v & 15) == 0 &&
                    A.kv_mul <= CH_MAXG && A.slot_count >= 64 &&
                    (int64_t)A.slot_count * A.value_stride * 4 < ((int64_t)1 << 31);
    A.sync = nullptr;
    // The streamed launch: the scores workgroups (as many per kv head, J, as
    // the CUs the chain workgroups leave, each scoring every J-th tile), then
    // the chain workgroups.  A scores workgroup takes about 4.5 us per tile
    // and the recurrence about 0.3 us, so with J >= 12 (or one tile each)
    // the scores keep up with it; otherwise separate launches.
    const int nc = A.n_kv * ((A.kv_mul + 3) / 4) * (A.vd / 16 + 1);
    const int J = std::max(1, std::min(ntl, (g.n_cu - nc) / A.n_kv));
    // J >= 12 also takes the Qwen2.5-14B shape (144 chain workgroups, J =
    // 14): at ctx 32768 its scores then run about level with the recurrence,
    // 171 us per layer against 193 for the separate launches
    static int jmin = -1;
    if (jmin < 0) {
        const char *e = getenv("RUSTY_HIP_STREAM_JMIN");
        jmin = e ? std::max(1, atoi(e)) : 12;
    }
    // A sliding window shorter than RUSTY_HIP_STREAM_MIN_WINDOW positions
    // (default 256) takes the separate launches: at gpt-oss's 128 positions
    // the streamed launch's start (scores published, polled, loaded) costs
    // more than the two extra launches (24.5 against 18.8 us per layer)
    static int min_window = -1;
    if (min_window < 0) {
        const char *e = getenv("RUSTY_HIP_STREAM_MIN_WINDOW");
        min_window = e ? std::max(0, atoi(e)) : 256;
    }
    const bool short_window = A.window > 0 && A.window < min_window;
    if (sync && s8 && c4 && A.n_tok == 0 && !A.lin && stream_enabled() && nc + 32 <= g.n_cu &&
        (J >= jmin || J >= ntl) && !short_window) {
        A.sync = sync;
        const int blocks = J * A.n_kv + nc;
        ProfScope ps("attn_exact_stream", s);
        if (A.hd == 128) rh_launch(attn_exact_stream_kernel<128>, dim3(blocks), dim3(64 * C4_WAVES), 0, s, A);
        else rh_launch(attn_exact_stream_kernel<64>, dim3(blocks), dim3(64 * C4_WAVES), 0, s, A);
        RH_LAUNCH_OK();
        if (den_out) *den_out = A.den;
        if (finish) {
            ProfScope ps2("attn_exact_finish", s);
            rh_launch(attn_exact_finish_kernel, dim3((n_out + 255) / 256), dim3(256), 0, s, A.out, A.den, A.vd, n_out, xq);
            RH_LAUNCH_OK();
        }
        return 1;
    }
    {
        ProfScope ps("attn_exact_scores", s);
        // many query tokens sharing the tile boundaries (no window, no ring
        // view): one K tile staging per block of tokens
        const bool mq = s8 && A.n_tok > 0 && !A.lin && A.window == 0 && !A.fuse_rope && A.q_tok % 4 == 0 &&
                        ((uintptr_t)A.q & 15) == 0;
        const unsigned nzb = (unsigned)((A.n_tok + mq_tokens(A.kv_mul) - 1) / mq_tokens(A.kv_mul));
        if (mq && A.hd == 128) {
            rh_launch(attn_exact_scores_mq_kernel<128>, dim3(ntl, A.n_kv, nzb), dim3(256), 0, s, A);
        } else if (mq) {
            rh_launch(attn_exact_scores_mq_kernel<64>, dim3(ntl, A.n_kv, nzb), dim3(256), 0, s, A);
        } else if (s8 && A.hd == 128) {
            rh_launch(attn_exact_scores8_kernel<128>, dim3(ntl, A.n_kv, nz), dim3(256), 0, s, A);
        } else if (s8) {
            rh_launch(attn_exact_scores8_kernel<64>, dim3(ntl, A.n_kv, nz), dim3(256), 0, s, A);
        } else {
            size_t lds = ((size_t)A.kv_mul * A.hd + (size_t)EX_TILE * (A.hd + 8) + (size_t)A.kv_mul * EX_TILE) *
                         sizeof(float);
            rh_launch(attn_exact_scores_kernel, dim3(ntl, A.n_kv, nz), dim3(256), lds, s, A);
        }
        RH_LAUNCH_OK();
    }
    if (!c4 || A.n_tok > 0) {
        ProfScope ps("attn_exact_coef", s);
        rh_launch(attn_exact_coef_kernel, dim3((ntl + 3) / 4, A.n_heads, nz), dim3(256), 0, s, A);
        RH_LAUNCH_OK();
    }
    {
        ProfScope ps("attn_exact_chain", s);
        if (c4 && A.n_tok > 0) {
            // many query tokens: one independent wave per task, no LDS ring;
            // four tokens per wave where they share the range start and the
            // transposed V copy covers the last token's range
            const int tasks = A.n_kv * ((A.kv_mul + 3) / 4) * (A.vd / 16 + 1);
            const int64_t ctx_last = (int64_t)A.pos0 + A.n_tok - A.start_t;
            const bool tok4 = chain_tok4_enabled() && A.vt != nullptr && A.window == 0 && !A.lin &&
                              (A.start_t & 3) == 0 && A.pos0 >= A.start_t &&
                              A.pos0 + A.n_tok - 1 < A.slot_count &&
                              A.start_t + (ctx_last + EX_TILE - 1) / EX_TILE * EX_TILE <= A.vt_stride &&
                              (int64_t)A.n_heads * A.cap < (1ll << 28) &&
                              A.tok_scratch < (1ll << 27);  // byte offsets within 31 bits
            if (tok4) {
                rh_launch(attn_exact_chain_tok4_kernel, dim3((tasks + 3) / 4, 1, (A.n_tok + 3) / 4), dim3(256), 0,
                          s, A);
            } else {
                rh_launch(attn_exact_chain_tok_kernel, dim3((tasks + 3) / 4, 1, nz), dim3(256), 0, s, A);
            }
        } else if (c4) {
            const int blocks = A.n_kv * ((A.kv_mul + 3) / 4) * (A.vd / 16 + 1);
            rh_launch(attn_exact_chain4_kernel, dim3(blocks, 1, nz), dim3(64 * C4_WAVES), 0, s, A);
        } else {
            rh_launch(attn_exact_chain_kernel, dim3(A.n_heads, (A.vd + 63) / 64, nz), dim3(64), 0, s, A);
        }
        RH_LAUNCH_OK();
    }
    if (den_out) *den_out = A.den;
    if (finish) {
        ProfScope ps("attn_exact_finish", s);
        rh_launch(attn_exact_finish_kernel, dim3((n_out + 255) / 256), dim3(256), 0, s, A.out, A.den, A.vd,
                           n_out, xq);
        RH_LAUNCH_OK();
    }
    return 1;
}

// ---- batched K-quant products (prefill) ------------------------------------------
// Q8_K activations of T tokens in one buffer: quants [T][K], then the scales
// token-minor [K/256][ldx] with ldx = T rounded up to the 64-token tile, so the
// product kernel reads four tokens' scales per 16-byte load without a bound.
struct BatchXq {
    int8_t *qs;
    float *dx;
    int ldx;
};
static int64_t batch_ldx(int T) { return ((int64_t)T + 63) / 64 * 64; }
static size_t batch_xq_bytes(int T, int K) { return (size_t)T * K + (size_t)(K / 256) * batch_ldx(T) * 4 + 256; }
static BatchXq batch_xq_at(int8_t *buf, int T, int K) {
    BatchXq b;
    b.qs = buf;
    b.dx = (float *)(buf + ((size_t)T * K + 255) / 256 * 256);
    b.ldx = (int)batch_ldx(T);
    return b;
}

static int quantize_batch_enqueue(const float *x, int ldxf, int T, int K, const BatchXq &b, hipStream_t s) {
    if (K % 256 != 0 || T <= 0) return 0;
    ProfScope ps("quantize_q8k_batch", s);
    rh_launch(quantize_q8k_batch_kernel, dim3((unsigned)(K / 256), (unsigned)T), dim3(256), 0, s, x, K, ldxf, b.qs,
              b.dx, b.ldx);
    RH_LAUNCH_OK();
    return 1;
}

// y[t * ldy + r] (=, or += with epi EPI_ADD) row r of W times token t, plus
// bias[r] when given; rows of one wave tile are 32 weight rows, a workgroup
// holds 4 tiles and covers 64 tokens.
static int gemm_kq_enqueue(const DevW &W, const BatchXq &b, int T, float *y, int ldy, int epi, const float *bias,
                           hipStream_t s, const char *prof_name = nullptr) {
    if ((W.fmt != 12 && W.fmt != 14) || W.cols % 256 != 0 || W.stride % 16 != 0 || T <= 0 || ldy < W.rows)
        return 0;
    GemmArgs A;
    memset(&A, 0, sizeof(A));
    A.w = W.p;
    A.row_stride = W.stride;
    A.rows = W.rows;
    A.K = W.cols;
    A.T = T;
    A.epi = epi;
    A.xq = b.qs;
    A.dx = b.dx;
    A.ldx = b.ldx;
    A.ldy = ldy;
    A.y = y;
    A.bias = bias;
    // 32 tokens per workgroup: a 64-token tile needs twice the registers
    // (two waves per SIMD) and measured slower (the smaller grids lose more
    // than the 14336-row products gain).
    // RUSTY_HIP_GEMM_KSPLIT: 0 never, 2 always, else (default) the K-split
    // kernel for Q6_K (whose row-tile kernel holds 256 registers, one wave
    // per SIMD) and for Q4_K when the row-tile grid would hold fewer
    // workgroups than CUs (the 1024-row k projection of an 8B-class model;
    // the 4096-row ones measured faster on the row-tile kernel)
    static int ksm = -1;
    if (ksm < 0) {
        const char *e = getenv("RUSTY_HIP_GEMM_KSPLIT");
        ksm = e ? atoi(e) : 1;
    }
    const int64_t row_tiles = (W.rows + 127) / 128;
    const int tok = 32;
    const int64_t tok_tiles = (T + tok - 1) / tok;
    const bool ks = ksm == 2 || (ksm == 1 && (W.fmt == 14 || row_tiles * tok_tiles < (int64_t)g.n_cu));
    ProfScope ps(prof_name ? prof_name : (W.fmt == 12 ? "gemm_q4k_mfma" : "gemm_q6k_mfma"), s);
    if (ks) {
        const dim3 grid((unsigned)((W.rows + 31) / 32), (unsigned)tok_tiles);
        if (W.fmt == 12)
            rh_launch(gemm_kq_mfma_ks_kernel<F_Q4_K>, grid, dim3(256), 0, s, A);
        else
            rh_launch(gemm_kq_mfma_ks_kernel<F_Q6_K>, grid, dim3(256), 0, s, A);
        RH_LAUNCH_OK();
        return 1;
    }
    const dim3 grid((unsigned)row_tiles, (unsigned)tok_tiles);
    const uint32_t lds = 2u * tok * GEMM_XS;
    if (W.fmt == 12)
        rh_launch(gemm_kq_mfma_kernel<F_Q4_K, 1>, grid, dim3(256), lds, s, A);
    else
        rh_launch(gemm_kq_mfma_kernel<F_Q6_K, 1>, grid, dim3(256), lds, s, A);
    RH_LAUNCH_OK();
    return 1;
}

// ---- per-op exports ------------------------------------------------------------------
static int stage_x(const float *x, size_t n) {
    if (!ensure(&g.x, &g.x_cap, n)) return 0;
    RH_CHECK(hipMemcpyAsync(g.x, x, n * sizeof(float), hipMemcpyHostToDevice, g.s));
    return 1;
}

// y_i = W_i x for up to 3 matrices sharing x (cols), each of its own type.
static int matvec_n(int n, const int *fmts, const uint8_t *const *w, const uintptr_t *wl, const uintptr_t *rows,
                    const float *x, uintptr_t cols, float *const *outs) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !x || cols == 0) return 0;
    MatSpec ms[3];
    size_t total = 0;
    for (int i = 0; i < n; i++) {
        if (!w[i] || !outs[i] || rows[i] == 0) return 0;
        if (!cat_of(fmts[i], (int)cols)) return 0;
        if (!get_weight(w[i], wl[i], (int64_t)rows[i], (int64_t)cols, fmts[i], &ms[i].w)) return 0;
        total += rows[i];
    }
    if (!stage_x(x, cols)) return 0;
    if (!ensure(&g.y, &g.y_cap, total)) return 0;
    size_t off = 0;
    for (int i = 0; i < n; i++) {
        ms[i].y = g.y + off;
        ms[i].bias = nullptr;
        off += rows[i];
    }
    bool need_q = false;
    for (int i = 0; i < n; i++)
        if (cat_of(fmts[i], (int)cols) != CAT_F32) need_q = true;
    if (need_q) {
        if (!ensure_xq(&g.xq, &g.xq_cap, cols)) return 0;
        if (!launch_quant(g.x, (int)cols, g.xq, g.s)) return 0;
    }
    if (!gemv_multi(ms, n, (int)cols, EPI_STORE, g.xq, g.x, g.s)) return 0;
    off = 0;
    for (int i = 0; i < n; i++) {
        RH_CHECK(hipMemcpyAsync(outs[i], g.y + off, rows[i] * sizeof(float), hipMemcpyDeviceToHost, g.s));
        off += rows[i];
    }
    RH_CHECK(hipStreamSynchronize(g.s));
    prof_drain();
    return 1;
}

static int ffn_device(const DevW &gate, const DevW &up, const DevW &down, int in_cols, const XQ &xq_in,
                      const float *x_in, float *y, int epi) {
    int hidden = gate.rows;
    if (!ensure(&g.hid, &g.hid_cap, (size_t)hidden * 3)) return 0;
    float *hbuf = g.hid, *tg = g.hid + hidden, *tu = g.hid + 2 * hidden;
    if (!gemv_swiglu(gate, up, in_cols, xq_in, x_in, hbuf, tg, tu, g.s)) return 0;
    bool need_q = cat_of(down.fmt, hidden) != CAT_F32;
    if (need_q) {
        if (!ensure_xq(&g.xq2, &g.xq2_cap, hidden)) return 0;
        if (!launch_quant(hbuf, hidden, g.xq2, g.s)) return 0;
    }
    MatSpec md = {down, y, nullptr};
    return gemv_multi(&md, 1, hidden, epi, g.xq2, hbuf, g.s);
}

// Routed MoE block (forward_gpt_oss_into, src/model.rs:6846-6898) on the
// device: router GEMV (+ bias), top-k + softmax, the k experts' gate and up
// rows in one launch (expert read on the device), SwiGLU with biases, the k
// down products in one launch (each with its own activation), then the
// combine.  Experts: rows of all experts stacked expert-major; f32-activation
// formats (MXFP4, Q8_0 with K % 256 != 0).  Scratch lives in `buf`
// (moe_scratch_floats); sel/prob are int32/f32 slots [k] inside it.
static size_t moe_scratch_floats(int n_exp, int k, int dim, int hidden) {
    return (size_t)64 + n_exp + 2 * 8 + (size_t)2 * k * hidden + (size_t)k * dim;
}
struct MoeDev {
    DevW router, gate, up, down;
    const float *router_bias, *gb, *ub, *db;  // device, may be null (router_bias: per expert; others [n_exp][rows])
    int gb_stride, ub_stride, db_stride;      // floats between expert bias rows
    int n_exp, k, dim, hidden;
};
// xq: the Q8_K form of xn for the router's integer path when dim is a whole
// number of 256-blocks; an empty XQ quantizes xn here into a buffer this call
// may allocate (so not under graph capture).
// norm_w: xn is first built as RMSNorm(norm_x) with norm_w (rms_norm_into),
// by the router launch's prologue where the router takes the Q8_0
// f32-activation kernel, else by a standalone RMSNorm launch.
static int moe_ffn_enqueue(const MoeDev &M, float *xn, const XQ &xq, float *moe_out, float *x_add, float *buf,
                           hipStream_t s, int32_t **sel_out = nullptr, float **prob_out = nullptr,
                           const float *norm_x = nullptr, const float *norm_w = nullptr, float norm_eps = 0.0f) {
    const int k = M.k, dim = M.dim, hidden = M.hidden;
    if (k < 1 || k > 8 || M.n_exp > 64 || k > M.n_exp) return 0;
    if (cat_of(M.gate.fmt, dim) != CAT_F32 || M.up.fmt != M.gate.fmt || cat_of(M.down.fmt, hidden) != CAT_F32)
        return 0;
    float *logits = buf;                        // [64]
    int32_t *sel = (int32_t *)(buf + 64);       // [8]
    float *prob = buf + 72;                     // [8]
    float *gate = buf + 80 + M.n_exp;           // [k][hidden]
    float *up = gate + (size_t)k * hidden;      // [k][hidden]
    float *proj = up + (size_t)k * hidden;      // [k][dim]
    gate = (float *)(((uintptr_t)gate + 15) & ~(uintptr_t)15);
    up = gate + (size_t)k * hidden;
    proj = up + (size_t)k * hidden;
    static int norm_fuse = -1;
    if (norm_fuse < 0) {
        const char *e = getenv("RUSTY_HIP_MOE_NORM_FUSE");
        norm_fuse = (e && e[0] == '0') ? 0 : 1;
    }
    if (norm_w && norm_fuse && M.router.fmt == F_Q8_0 && cat_of(M.router.fmt, dim) == CAT_F32 && dim % 4 == 0 &&
        dim <= 3072 && ((uintptr_t)norm_x & 15) == 0 && ((uintptr_t)norm_w & 15) == 0 && ((uintptr_t)xn & 15) == 0) {
        GemvArgs A;
        memset(&A, 0, sizeof(A));
        A.K = dim;
        A.epi = EPI_STORE;
        A.x = norm_x;
        A.n_mats = 1;
        A.m[0].w = M.router.p;
        A.m[0].row_stride = M.router.stride;
        A.m[0].rows = M.router.rows;
        A.m[0].fmt = M.router.fmt;
        A.m[0].y = logits;
        A.m[0].bias = M.router_bias;
        A.n_tiles = (M.router.rows + 7) / 8;
        A.norm_w = norm_w;
        A.norm_eps = norm_eps;
        A.norm_out = xn;
        ProfScope ps("gemv_f32x", s);
        rh_launch(gemv_q8_0_f32x_kernel<true>, dim3(A.n_tiles), dim3(64), (uint32_t)(A.K * sizeof(float)), s, A);
        RH_LAUNCH_OK();
    } else {
        // the norm also writes the Q8_K form into the caller's buffer when the
        // router takes the integer path (no allocation: this may be captured)
        if (norm_w && !launch_rmsnorm(norm_x, norm_w, norm_eps, dim, xn, (dim % 256 == 0 && xq.qs) ? &xq : nullptr, s))
            return 0;
        MatSpec mr = {M.router, logits, M.router_bias};
        ActSpec a;
        memset(&a, 0, sizeof(a));
        a.mode = (dim % 256 == 0 && !xq.qs) ? ACT_QUANT : ACT_XQ;
        a.x = (float *)xn;
        if (a.mode == ACT_QUANT && !ensure_xq(&g.xq, &g.xq_cap, dim)) return 0;
        a.xq = a.mode == ACT_QUANT ? g.xq : (dim % 256 == 0 ? xq : XQ{});
        if (!gemv_multi_act(&mr, 1, dim, EPI_STORE, a, s)) return 0;
    }
    // MXFP4 gate/up with as many 32-row tiles as the one-wave kernel takes:
    // SwiGLU (and the biases) in its epilogue, no moe_swiglu launch, and the
    // top-k selection in every workgroup, no moe_topk launch
    static int swi_fuse = -1;
    if (swi_fuse < 0) {
        const char *e = getenv("RUSTY_HIP_MOE_SWIGLU_FUSE");
        swi_fuse = (e && e[0] == '0') ? 0 : 1;
    }
    const int swi_tiles = k * ((hidden + 31) / 32);
    const bool swi = swi_fuse && M.gate.fmt == F_MXFP4 && 2 * k <= GEMV_MAX_MATS && M.up.stride == M.gate.stride &&
                     swi_tiles > mx_serial_per_cu() * g.n_cu && mx_fused_fits(dim);
    if (!swi) {
        ProfScope ps("moe_topk", s);
        rh_launch(moe_topk_kernel, dim3(1), dim3(64), 0, s, (const float *)logits, M.n_exp, k, sel, prob);
        RH_LAUNCH_OK();
    }
    auto expert_mat = [&](const DevW &W, int rows, int r, float *y, const float *x) {
        GemvMat m;
        memset(&m, 0, sizeof(m));
        m.w = W.p;
        m.row_stride = W.stride;
        m.rows = rows;
        m.fmt = W.fmt;
        m.y = y;
        m.x = x;
        m.sel = sel + r;
        m.sel_w = (int64_t)rows * W.stride;
        return m;
    };
    auto launch = [&](GemvArgs &A, int rows_per_tile) {
        int tiles = 0;
        for (int i = 0; i < A.n_mats; i++) {
            A.m[i].tile_begin = tiles;
            tiles += (A.m[i].rows + rows_per_tile - 1) / rows_per_tile;
        }
        A.n_tiles = tiles;
        return A.m[0].fmt == 8 ? launch_f32x<F_Q8_0>(A, s) : launch_f32x<F_MXFP4>(A, s);
    };
    const int rpt_in = M.gate.fmt == 8 ? 8 : 64, rpt_down = M.down.fmt == 8 ? 8 : 64;
    if (swi) {
        GemvArgs A;
        memset(&A, 0, sizeof(A));
        A.K = dim;
        A.epi = EPI_STORE;
        A.x = xn;
        A.n_mats = 2 * k;
        for (int r = 0; r < k; r++) {
            A.m[r] = expert_mat(M.gate, hidden, r, gate + (size_t)r * hidden, nullptr);
            A.m[r].bias = M.gb;
            A.m[r].sel_b = M.gb_stride;
            A.m[r].tile_begin = r * ((hidden + 31) / 32);
            A.m[k + r] = expert_mat(M.up, hidden, r, up + (size_t)r * hidden, nullptr);
            A.m[k + r].bias = M.ub;
            A.m[k + r].sel_b = M.ub_stride;
        }
        A.n_tiles = swi_tiles;
        A.topk_logits = logits;
        A.topk_n = M.n_exp;
        A.topk_k = k;
        A.topk_sel = sel;
        A.topk_prob = prob;
        ProfScope ps("gemv_mxfp4", s);
        rh_launch(gemv_mxfp4_fused_kernel<true>, dim3(A.n_tiles), dim3(64), mx_fused_x_bytes(A.K), s, A);
        RH_LAUNCH_OK();
    } else {
    {
        GemvArgs A;
        memset(&A, 0, sizeof(A));
        A.K = dim;
        A.epi = EPI_STORE;
        A.x = xn;
        A.n_mats = 2 * k;
        for (int r = 0; r < k; r++) {
            A.m[r] = expert_mat(M.gate, hidden, r, gate + (size_t)r * hidden, nullptr);
            A.m[k + r] = expert_mat(M.up, hidden, r, up + (size_t)r * hidden, nullptr);
        }
        if (!launch(A, rpt_in)) return 0;
    }
    {
        ProfScope ps("moe_swiglu", s);
        rh_launch(moe_swiglu_kernel, dim3((hidden + 255) / 256, k), dim3(256), 0, s, gate, (const float *)up, hidden, k,
                  (const int32_t *)sel, M.gb, M.gb_stride, M.ub, M.ub_stride);
        RH_LAUNCH_OK();
    }
    }
    {
        GemvArgs A;
        memset(&A, 0, sizeof(A));
        A.K = hidden;
        A.epi = EPI_STORE;
        A.n_mats = k;
        for (int r = 0; r < k; r++)
            A.m[r] = expert_mat(M.down, dim, r, proj + (size_t)r * dim, gate + (size_t)r * hidden);
        if (!launch(A, rpt_down)) return 0;
    }
    {
        ProfScope ps("moe_combine", s);
        rh_launch(moe_combine_kernel, dim3((dim + 255) / 256), dim3(256), 0, s, (const float *)proj, dim, k,
                  (const int32_t *)sel, (const float *)prob, M.db, M.db_stride, moe_out, x_add);
        RH_LAUNCH_OK();
    }
    if (sel_out) *sel_out = sel;
    if (prob_out) *prob_out = prob;
    return 1;
}

}  // namespace rh

using namespace rh;

namespace rh {
void r_invalidate_graphs_extern();
}

extern "C" {

int rusty_hip_available(void) {
    std::lock_guard<std::mutex> lk(g.mu);
    return init_locked();
}

int rusty_hip_matvec(uint32_t t, const uint8_t *w, uintptr_t wl, const float *x, uintptr_t rows, uintptr_t cols,
                     float *out) {
    int f[1] = {(int)t};
    const uint8_t *ws[1] = {w};
    uintptr_t wls[1] = {wl}, rs[1] = {rows};
    float *os[1] = {out};
    return matvec_n(1, f, ws, wls, rs, x, cols, os);
}

int rusty_hip_q4k_matvec(const uint8_t *w, uintptr_t wl, const float *x, uintptr_t rows, uintptr_t cols, float *out) {
    return rusty_hip_matvec(12, w, wl, x, rows, cols, out);
}
int rusty_hip_q6k_matvec(const uint8_t *w, uintptr_t wl, const float *x, uintptr_t rows, uintptr_t cols, float *out) {
    return rusty_hip_matvec(14, w, wl, x, rows, cols, out);
}
int rusty_hip_q8_0_matvec(const uint8_t *w, uintptr_t wl, const float *x, uintptr_t rows, uintptr_t cols, float *out) {
    return rusty_hip_matvec(8, w, wl, x, rows, cols, out);
}
int rusty_hip_mxfp4_matvec(const uint8_t *w, uintptr_t wl, const float *x, uintptr_t rows, uintptr_t cols,
                           float *out) {
    return rusty_hip_matvec(39, w, wl, x, rows, cols, out);
}

static int mv2(int fa, int fb, const uint8_t *wa, uintptr_t la, uintptr_t ra, const uint8_t *wb, uintptr_t lb,
               uintptr_t rb, const float *x, uintptr_t cols, float *oa, float *ob) {
    int f[2] = {fa, fb};
    const uint8_t *ws[2] = {wa, wb};
    uintptr_t wls[2] = {la, lb}, rs[2] = {ra, rb};
    float *os[2] = {oa, ob};
    return matvec_n(2, f, ws, wls, rs, x, cols, os);
}
static int mv3(int fa, int fb, int fc, const uint8_t *wa, uintptr_t la, uintptr_t ra, const uint8_t *wb,
               uintptr_t lb, uintptr_t rb, const uint8_t *wc, uintptr_t lc, uintptr_t rc, const float *x,
               uintptr_t cols, float *oa, float *ob, float *oc) {
    int f[3] = {fa, fb, fc};
    const uint8_t *ws[3] = {wa, wb, wc};
    uintptr_t wls[3] = {la, lb, lc}, rs[3] = {ra, rb, rc};
    float *os[3] = {oa, ob, oc};
    return matvec_n(3, f, ws, wls, rs, x, cols, os);
}

int rusty_hip_q6k_matvec2(const uint8_t *wa, uintptr_t la, uintptr_t ra, const uint8_t *wb, uintptr_t lb,
                          uintptr_t rb, const float *x, uintptr_t cols, float *oa, float *ob) {
    return mv2(14, 14, wa, la, ra, wb, lb, rb, x, cols, oa, ob);
}
int rusty_hip_q6k_matvec3(const uint8_t *wa, uintptr_t la, uintptr_t ra, const uint8_t *wb, uintptr_t lb,
                          uintptr_t rb, const uint8_t *wc, uintptr_t lc, uintptr_t rc, const float *x, uintptr_t cols,
                          float *oa, float *ob, float *oc) {
    return mv3(14, 14, 14, wa, la, ra, wb, lb, rb, wc, lc, rc, x, cols, oa, ob, oc);
}
int rusty_hip_q4k_matvec2(const uint8_t *wa, uintptr_t la, uintptr_t ra, const uint8_t *wb, uintptr_t lb,
                          uintptr_t rb, const float *x, uintptr_t cols, float *oa, float *ob) {
    return mv2(12, 12, wa, la, ra, wb, lb, rb, x, cols, oa, ob);
}
int rusty_hip_q4k_matvec3(const uint8_t *wa, uintptr_t la, uintptr_t ra, const uint8_t *wb, uintptr_t lb,
                          uintptr_t rb, const uint8_t *wc, uintptr_t lc, uintptr_t rc, const float *x, uintptr_t cols,
                          float *oa, float *ob, float *oc) {
    return mv3(12, 12, 12, wa, la, ra, wb, lb, rb, wc, lc, rc, x, cols, oa, ob, oc);
}
int rusty_hip_q4k_q4k_q6k_matvec3(const uint8_t *wa, uintptr_t la, uintptr_t ra, const uint8_t *wb, uintptr_t lb,
                                  uintptr_t rb, const uint8_t *wc, uintptr_t lc, uintptr_t rc, const float *x,
                                  uintptr_t cols, float *oa, float *ob, float *oc) {
    return mv3(12, 12, 14, wa, la, ra, wb, lb, rb, wc, lc, rc, x, cols, oa, ob, oc);
}
int rusty_hip_mxfp4_matvec2(const uint8_t *wa, uintptr_t la, uintptr_t ra, const uint8_t *wb, uintptr_t lb,
                            uintptr_t rb, const float *x, uintptr_t cols, float *oa, float *ob) {
    return mv2(39, 39, wa, la, ra, wb, lb, rb, x, cols, oa, ob);
}

int rusty_hip_q4k_q4k_q6k_ffn(const uint8_t *gw, uintptr_t gl, const uint8_t *uw, uintptr_t ul, const uint8_t *dw,
                              uintptr_t dl, const float *x, uintptr_t in_cols, uintptr_t hidden_rows,
                              uintptr_t down_rows, uintptr_t down_cols, float *out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !gw || !uw || !dw || !x || !out || in_cols == 0 || hidden_rows == 0 || down_rows == 0 ||
        down_cols == 0 || hidden_rows != down_cols || in_cols % 256 != 0 || down_cols % 256 != 0)
        return 0;
    DevW G, U, D;
    if (!get_weight(gw, gl, hidden_rows, in_cols, 12, &G) || !get_weight(uw, ul, hidden_rows, in_cols, 12, &U) ||
        !get_weight(dw, dl, down_rows, down_cols, 14, &D))
        return 0;
    if (!stage_x(x, in_cols) || !ensure(&g.y, &g.y_cap, down_rows)) return 0;
    if (!ensure_xq(&g.xq, &g.xq_cap, in_cols) || !launch_quant(g.x, (int)in_cols, g.xq, g.s)) return 0;
    if (!ffn_device(G, U, D, (int)in_cols, g.xq, g.x, g.y, EPI_STORE)) return 0;
    RH_CHECK(hipMemcpyAsync(out, g.y, down_rows * sizeof(float), hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    prof_drain();
    return 1;
}

int rusty_hip_mistral_post_attention_ffn(const uint8_t *ow, uintptr_t ol, const uint8_t *gw, uintptr_t gl,
                                         const uint8_t *uw, uintptr_t ul, const uint8_t *dw, uintptr_t dl, float *x,
                                         uintptr_t dim, const float *attn_out, uintptr_t attn_cols,
                                         const float *ffn_norm, float eps, uintptr_t hidden_rows,
                                         uintptr_t down_rows, uintptr_t down_cols) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !ow || !gw || !uw || !dw || !x || !attn_out || !ffn_norm || dim == 0 || attn_cols == 0 ||
        hidden_rows == 0 || down_rows == 0 || down_cols == 0 || down_rows != dim || hidden_rows != down_cols ||
        dim % 256 != 0 || attn_cols % 256 != 0 || down_cols % 256 != 0)
        return 0;
    DevW O, G, U, D;
    if (!get_weight(ow, ol, dim, attn_cols, 12, &O) || !get_weight(gw, gl, hidden_rows, dim, 12, &G) ||
        !get_weight(uw, ul, hidden_rows, dim, 12, &U) || !get_weight(dw, dl, down_rows, down_cols, 14, &D))
        return 0;
    // device layout in g.y: [x (dim) | attn (attn_cols) | norm w (dim) | xn (dim)]
    if (!ensure(&g.y, &g.y_cap, 3 * dim + attn_cols)) return 0;
    float *dx = g.y, *da = g.y + dim, *dw_ = da + attn_cols, *dxn = dw_ + dim;
    RH_CHECK(hipMemcpyAsync(dx, x, dim * 4, hipMemcpyHostToDevice, g.s));
    RH_CHECK(hipMemcpyAsync(da, attn_out, attn_cols * 4, hipMemcpyHostToDevice, g.s));
    RH_CHECK(hipMemcpyAsync(dw_, ffn_norm, dim * 4, hipMemcpyHostToDevice, g.s));
    if (!ensure_xq(&g.xq, &g.xq_cap, std::max(dim, attn_cols))) return 0;
    if (!launch_quant(da, (int)attn_cols, g.xq, g.s)) return 0;
    MatSpec mo = {O, dx, nullptr};
    if (!gemv_multi(&mo, 1, (int)attn_cols, EPI_ADD, g.xq, da, g.s)) return 0;
    if (!launch_rmsnorm(dx, dw_, eps, (int)dim, dxn, &g.xq, g.s)) return 0;
    if (!ffn_device(G, U, D, (int)dim, g.xq, dxn, dx, EPI_ADD)) return 0;
    RH_CHECK(hipMemcpyAsync(x, dx, dim * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    prof_drain();
    return 1;
}

}  // extern "C"

namespace rh {
// Argument checks of rusty_metal_attention (src/metal.rs:277-299; *_len are
// byte lengths, metal_backend.m:2082-2086), shared by both attention exports.
static bool attn_export_args_ok(const float *query, uintptr_t query_len, const float *keys, uintptr_t keys_len,
                                const float *values, uintptr_t values_len, const float *sinks, uintptr_t sinks_len,
                                const float *out, uintptr_t out_len, uintptr_t heads, uintptr_t kv_mul,
                                uintptr_t head_dim, uintptr_t value_dim, uintptr_t key_stride, uintptr_t value_stride,
                                uintptr_t slot_count, uintptr_t start_t, uintptr_t end_t, int use_sink) {
    if (!query || !keys || !values || !out || heads == 0 || kv_mul == 0 || head_dim == 0 || value_dim == 0 ||
        slot_count == 0 || head_dim > 256 || value_dim > 256)
        return false;
    if (heads % kv_mul != 0 || !attn_supported((int)head_dim, (int)value_dim, (int)kv_mul)) return false;
    if (key_stride % 4 != 0 || value_stride % 4 != 0) return false;
    const size_t n_kv = heads / kv_mul;
    if (key_stride < n_kv * head_dim || value_stride < n_kv * value_dim) return false;
    if (query_len < heads * head_dim * 4 || keys_len < slot_count * key_stride * 4 ||
        values_len < slot_count * value_stride * 4 || out_len < heads * value_dim * 4 ||
        (use_sink && (!sinks || sinks_len < heads * 4)))
        return false;
    // positions and slots travel as int32 in the kernels
    if (end_t >= (uintptr_t)INT32_MAX || slot_count >= (uintptr_t)INT32_MAX) return false;
    return true;
}

// One attention call over device buffers on the library stream: the scratch
// it needs (floats), and the launches.  Exact mode: scores, coefficients and
// masks of a cap-position range (exact_scratch_floats); split-K: the
// per-chunk partials.
struct AttnCall {
    AttnArgs A;
    bool fast;
    int cap;
    size_t scratch_floats;
};
static AttnCall attn_call_plan(const float *q, const float *k, const float *v, const float *sinks, float *out,
                               uintptr_t heads, uintptr_t kv_mul, uintptr_t head_dim, uintptr_t value_dim,
                               uintptr_t key_stride, uintptr_t value_stride, uintptr_t slot_count, uintptr_t start_t,
                               uintptr_t end_t, float scale) {
    AttnCall C;
    memset(&C, 0, sizeof(C));
    AttnArgs &A = C.A;
    A.q = q;
    A.k = k;
    A.v = v;
    A.sinks = sinks;
    A.out = out;
    A.n_heads = (int)heads;
    A.n_kv = (int)(heads / kv_mul);
    A.kv_mul = (int)kv_mul;
    A.hd = (int)head_dim;
    A.vd = (int)value_dim;
    A.key_stride = (int64_t)key_stride;
    A.value_stride = (int64_t)value_stride;
    A.slot_count = (int)slot_count;
    A.start_t = (int)start_t;
    A.end_t = (int)end_t;
    A.scale = scale;
    const int ctx = (int)(end_t - start_t + 1);
    A.n_chunks = attn_chunks(A.n_kv, ctx);
    C.fast = attn_fast_mode() != 0;
    C.cap = (ctx + 63) / 64 * 64;
    C.scratch_floats = C.fast ? (size_t)A.n_kv * A.n_chunks * A.kv_mul * att_pstride(A.vd)
                              : exact_scratch_floats(A.n_kv, A.kv_mul, C.cap);
    return C;
}
static int attn_call_launch(AttnCall C, float *scratch, hipStream_t s) {
    const AttnArgs &A = C.A;
    if (C.fast) {
        C.A.part = scratch;
        return attn_launch(C.A, s);
    }
    AttnExactArgs E;
    memset(&E, 0, sizeof(E));
    E.q = A.q;
    E.k = A.k;
    E.v = A.v;
    E.sinks = A.sinks;
    E.out = A.out;
    E.n_heads = A.n_heads;
    E.n_kv = A.n_kv;
    E.kv_mul = A.kv_mul;
    E.hd = A.hd;
    E.vd = A.vd;
    E.key_stride = A.key_stride;
    E.value_stride = A.value_stride;
    E.slot_count = A.slot_count;
    E.start_t = A.start_t;
    E.end_t = A.end_t;
    E.scale = A.scale;
    E.cap = C.cap;
    return attn_exact_launch(E, scratch, XQ{}, s);
}
}  // namespace rh

extern "C" {

int rusty_hip_attention(const float *query, uintptr_t query_len, const float *keys, uintptr_t keys_len,
                        const float *values, uintptr_t values_len, const float *sinks, uintptr_t sinks_len, float *out,
                        uintptr_t out_len, uintptr_t heads, uintptr_t kv_mul, uintptr_t head_dim, uintptr_t value_dim,
                        uintptr_t key_stride, uintptr_t value_stride, uintptr_t slot_count, uintptr_t start_t,
                        uintptr_t end_t, float scale, int use_sink) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() ||
        !attn_export_args_ok(query, query_len, keys, keys_len, values, values_len, sinks, sinks_len, out, out_len,
                             heads, kv_mul, head_dim, value_dim, key_stride, value_stride, slot_count, start_t, end_t,
                             use_sink))
        return 0;
    if (start_t > end_t) {  // empty range: the reference leaves out untouched
        return 1;
    }
    // Upload only the slots the scan visits.
    size_t lo, n_slots;
    if (end_t < slot_count) {
        lo = start_t;
        n_slots = end_t - start_t + 1;
    } else {
        lo = 0;
        n_slots = slot_count;
    }
    size_t kfl = slot_count * key_stride, vfl = slot_count * value_stride;
    if (!ensure(&g.kv_k, &g.kv_cap, kfl + vfl)) return 0;
    g.kv_v = g.kv_k + kfl;
    RH_CHECK(hipMemcpyAsync(g.kv_k + lo * key_stride, keys + lo * key_stride, n_slots * key_stride * 4,
                            hipMemcpyHostToDevice, g.s));
    RH_CHECK(hipMemcpyAsync(g.kv_v + lo * value_stride, values + lo * value_stride, n_slots * value_stride * 4,
                            hipMemcpyHostToDevice, g.s));
    size_t qn = heads * head_dim, on = heads * value_dim;
    if (!ensure(&g.x, &g.x_cap, qn + heads) || !ensure(&g.y, &g.y_cap, on)) return 0;
    RH_CHECK(hipMemcpyAsync(g.x, query, qn * 4, hipMemcpyHostToDevice, g.s));
    if (use_sink) RH_CHECK(hipMemcpyAsync(g.x + qn, sinks, heads * 4, hipMemcpyHostToDevice, g.s));
    AttnCall C = attn_call_plan(g.x, g.kv_k, g.kv_v, use_sink ? g.x + qn : nullptr, g.y, heads, kv_mul, head_dim,
                                value_dim, key_stride, value_stride, slot_count, start_t, end_t, scale);
    float *scr;
    if (C.fast) {
        if (!ensure(&g.part, &g.part_cap, C.scratch_floats)) return 0;
        scr = g.part;
    } else {
        if (!ensure(&g.ex, &g.ex_cap, C.scratch_floats)) return 0;
        scr = g.ex;
    }
    if (!attn_call_launch(C, scr, g.s)) return 0;
    RH_CHECK(hipMemcpyAsync(out, g.y, on * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    prof_drain();
    return 1;
}

// rusty_hip_attention over device buffers with no allocation: the scratch is
// the static `scratch` array of this device (its address taken at init).
// Calls that overlap on one GPU share that array and race; each call
// writes every scratch word it later reads, so nothing needs clearing.
int rusty_hip_attention_noalloc(const float *query, uintptr_t query_len, const float *keys, uintptr_t keys_len,
                                const float *values, uintptr_t values_len, const float *sinks, uintptr_t sinks_len,
                                float *out, uintptr_t out_len, uintptr_t heads, uintptr_t kv_mul, uintptr_t head_dim,
                                uintptr_t value_dim, uintptr_t key_stride, uintptr_t value_stride,
                                uintptr_t slot_count, uintptr_t start_t, uintptr_t end_t, float scale, int use_sink) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() ||
        !attn_export_args_ok(query, query_len, keys, keys_len, values, values_len, sinks, sinks_len, out, out_len,
                             heads, kv_mul, head_dim, value_dim, key_stride, value_stride, slot_count, start_t, end_t,
                             use_sink))
        return 0;
    float *scr = g.noalloc[g.dev];
    if (!scr) return 0;
    if (start_t > end_t) return 1;  // empty range: out untouched, as the reference
    AttnCall C = attn_call_plan(query, keys, values, use_sink ? sinks : nullptr, out, heads, kv_mul, head_dim,
                                value_dim, key_stride, value_stride, slot_count, start_t, end_t, scale);
    if (C.scratch_floats * sizeof(float) > RH_NOALLOC_SCRATCH_BYTES) {
        fprintf(stderr,
                "[rusty_hip] rusty_hip_attention_noalloc: %zu bytes of scratch needed for %zu heads over %zu "
                "positions, above the fixed %u-byte maximum; call rusty_hip_attention instead\n",
                C.scratch_floats * sizeof(float), (size_t)heads, (size_t)(end_t - start_t + 1),
                (unsigned)RH_NOALLOC_SCRATCH_BYTES);
        return 0;
    }
    // the inputs may come from any stream of the caller's: all work already
    // submitted to the device completes first
    RH_CHECK(hipDeviceSynchronize());
    if (!attn_call_launch(C, scr, g.s)) return 0;
    RH_CHECK(hipStreamSynchronize(g.s));
    prof_drain();
    return 1;
}

int rusty_hip_attention_mode(int mode) {
    std::lock_guard<std::mutex> lk(g.mu);
    int prev = attn_fast_mode();
    if (mode == 0 || mode == 1) {
        if (mode != prev) {
            g.attn_fast = mode;
            r_invalidate_graphs_extern();
        }
    }
    return prev;
}

int rusty_hip_moe_ffn(const float *x, uintptr_t dim, const uint8_t *router_w, uintptr_t router_w_len,
                      uint32_t router_dt, const float *router_bias, uint32_t n_experts, uint32_t top_k,
                      const uint8_t *gate_w, uintptr_t gate_w_len, const uint8_t *up_w, uintptr_t up_w_len,
                      const uint8_t *down_w, uintptr_t down_w_len, uint32_t expert_dt, uintptr_t hidden,
                      const float *gate_bias, const float *up_bias, const float *down_bias, float *out,
                      int32_t *selected, float *probs) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !x || !router_w || !gate_w || !up_w || !down_w || !out || dim == 0 || hidden == 0 ||
        n_experts == 0 || n_experts > 64 || top_k == 0 || top_k > 8 || top_k > n_experts)
        return 0;
    MoeDev M;
    memset(&M, 0, sizeof(M));
    M.n_exp = (int)n_experts;
    M.k = (int)top_k;
    M.dim = (int)dim;
    M.hidden = (int)hidden;
    auto ggml_type = [](uint32_t t) { return (t == 8 || t == 12 || t == 14 || t == 39) ? (int)t : -1; };
    const int rdt = ggml_type(router_dt), edt = ggml_type(expert_dt);
    if (rdt < 0 || edt < 0) return 0;
    if (!get_weight(router_w, router_w_len, n_experts, dim, rdt, &M.router) ||
        !get_weight(gate_w, gate_w_len, (int64_t)n_experts * hidden, dim, edt, &M.gate) ||
        !get_weight(up_w, up_w_len, (int64_t)n_experts * hidden, dim, edt, &M.up) ||
        !get_weight(down_w, down_w_len, (int64_t)n_experts * dim, hidden, edt, &M.down))
        return 0;
    DevW rb, gb, ub, db;
    if (router_bias) {
        if (!get_weight((const uint8_t *)router_bias, n_experts * 4, 1, n_experts, 0, &rb)) return 0;
        M.router_bias = (const float *)rb.p;
    }
    if (gate_bias) {
        if (!get_weight((const uint8_t *)gate_bias, n_experts * hidden * 4, n_experts, hidden, 0, &gb)) return 0;
        M.gb = (const float *)gb.p;
        M.gb_stride = (int)(gb.stride / 4);
    }
    if (up_bias) {
        if (!get_weight((const uint8_t *)up_bias, n_experts * hidden * 4, n_experts, hidden, 0, &ub)) return 0;
        M.ub = (const float *)ub.p;
        M.ub_stride = (int)(ub.stride / 4);
    }
    if (down_bias) {
        if (!get_weight((const uint8_t *)down_bias, n_experts * dim * 4, n_experts, dim, 0, &db)) return 0;
        M.db = (const float *)db.p;
        M.db_stride = (int)(db.stride / 4);
    }
    if (!ensure(&g.x, &g.x_cap, dim) || !ensure(&g.y, &g.y_cap, dim) ||
        !ensure(&g.moe, &g.moe_cap, moe_scratch_floats(M.n_exp, M.k, M.dim, M.hidden) + 8))
        return 0;
    RH_CHECK(hipMemcpyAsync(g.x, x, dim * 4, hipMemcpyHostToDevice, g.s));
    int32_t *sel = nullptr;
    float *prob = nullptr;
    if (!moe_ffn_enqueue(M, g.x, XQ{}, g.y, nullptr, g.moe, g.s, &sel, &prob)) return 0;
    RH_CHECK(hipMemcpyAsync(out, g.y, dim * 4, hipMemcpyDeviceToHost, g.s));
    if (selected) RH_CHECK(hipMemcpyAsync(selected, sel, top_k * 4, hipMemcpyDeviceToHost, g.s));
    if (probs) RH_CHECK(hipMemcpyAsync(probs, prob, top_k * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    prof_drain();
    return 1;
}

__global__ void expf_kernel(const float *x, int n, float *out) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) out[i] = expf_glibc(x[i]);
}
int rusty_hip_debug_expf(const float *x, uintptr_t n, float *out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !x || !out || n == 0) return 0;
    if (!ensure(&g.x, &g.x_cap, n) || !ensure(&g.y, &g.y_cap, n)) return 0;
    RH_CHECK(hipMemcpyAsync(g.x, x, n * 4, hipMemcpyHostToDevice, g.s));
    rh_launch(expf_kernel, dim3(1024), dim3(256), 0, g.s, g.x, (int)n, g.y);
    RH_LAUNCH_OK();
    RH_CHECK(hipMemcpyAsync(out, g.y, n * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    return 1;
}

int rusty_hip_weight_cache_clear(void) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked()) return 0;
    wcache_clear();
    return 1;
}

int rusty_hip_sync(void) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked()) return 0;
    RH_CHECK(hipStreamSynchronize(g.s));
    prof_drain();
    return 1;
}

int rusty_hip_profile_enable(int on) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked()) return 0;
    prof_drain();
    g.prof.on = on != 0;
    if (on) {
        for (auto &t : g.prof.total_ms) t = 0.0;
        for (auto &c : g.prof.count) c = 0;
    }
    return 1;
}

int rusty_hip_profile_get(int i, char *name, double *total_ms, int64_t *count) {
    std::lock_guard<std::mutex> lk(g.mu);
    prof_drain();
    if (i < 0 || i >= (int)g.prof.names.size()) return 0;
    if (name) {
        strncpy(name, g.prof.names[i].c_str(), 63);
        name[63] = 0;
    }
    if (total_ms) *total_ms = g.prof.total_ms[i];
    if (count) *count = g.prof.count[i];
    return 1;
}

// ---- debug hooks ----------------------------------------------------------------------
int rusty_hip_debug_quantize_q8k(const float *x, uintptr_t n, int8_t *qs, float *d, int16_t *bsums) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !x || n == 0 || n % 256 != 0) return 0;
    if (!stage_x(x, n) || !ensure_xq(&g.xq, &g.xq_cap, n) || !launch_quant(g.x, (int)n, g.xq, g.s)) return 0;
    RH_CHECK(hipMemcpyAsync(qs, g.xq.qs, n, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipMemcpyAsync(d, g.xq.d, n / 256 * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipMemcpyAsync(bsums, g.xq.bsums, n / 32 * 2, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    return 1;
}

int rusty_hip_debug_dequant(uint32_t t, const uint8_t *w, uintptr_t wl, uintptr_t rows, uintptr_t cols, float *out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !w || !out) return 0;
    DevW W;
    if (!get_weight(w, wl, rows, cols, (int)t, &W)) return 0;
    if (!ensure(&g.y, &g.y_cap, rows * cols)) return 0;
    dim3 grid((unsigned)std::min<uintptr_t>((cols + 255) / 256, 64), (unsigned)rows);
    rh_launch(dequant_rows_kernel, grid, dim3(256), 0, g.s, W.p, W.stride, (int)rows, (int)cols, (int)t, g.y);
    RH_LAUNCH_OK();
    RH_CHECK(hipMemcpyAsync(out, g.y, rows * cols * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    return 1;
}

int rusty_hip_debug_block_ints(uint32_t t, const uint8_t *w, uintptr_t wl, uintptr_t rows, uintptr_t cols,
                               const float *x, int32_t *out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !w || !x || !out || cols % 256 != 0) return 0;
    if (t != 8 && t != 12 && t != 14) return 0;
    DevW W;
    if (!get_weight(w, wl, rows, cols, (int)t, &W)) return 0;
    if (!stage_x(x, cols) || !ensure_xq(&g.xq, &g.xq_cap, cols) || !launch_quant(g.x, (int)cols, g.xq, g.s)) return 0;
    size_t n = (t == 8) ? rows * (cols / 32) : (t == 12 ? rows * (cols / 256) * 2 : rows * (cols / 256));
    if (!ensure(&g.ibuf, &g.ibuf_cap, n)) return 0;
    rh_launch(block_ints_kernel, dim3((unsigned)rows), dim3(64), 0, g.s, W.p, W.stride, (int)rows, (int)cols,
                       (int)t, g.xq, g.ibuf);
    RH_LAUNCH_OK();
    RH_CHECK(hipMemcpyAsync(out, g.ibuf, n * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    return 1;
}

int rusty_hip_debug_rmsnorm(const float *x, const float *w, float eps, uintptr_t n, float *out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !x || !w || !out || n == 0) return 0;
    if (!ensure(&g.x, &g.x_cap, 2 * n) || !ensure(&g.y, &g.y_cap, n)) return 0;
    RH_CHECK(hipMemcpyAsync(g.x, x, n * 4, hipMemcpyHostToDevice, g.s));
    RH_CHECK(hipMemcpyAsync(g.x + n, w, n * 4, hipMemcpyHostToDevice, g.s));
    if (!launch_rmsnorm(g.x, g.x + n, eps, (int)n, g.y, nullptr, g.s)) return 0;
    RH_CHECK(hipMemcpyAsync(out, g.y, n * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    return 1;
}

int rusty_hip_debug_silu_mul(const float *gt, const float *up, uintptr_t n, float *out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !gt || !up || !out || n == 0) return 0;
    if (!ensure(&g.x, &g.x_cap, 2 * n) || !ensure(&g.y, &g.y_cap, n)) return 0;
    RH_CHECK(hipMemcpyAsync(g.x, gt, n * 4, hipMemcpyHostToDevice, g.s));
    RH_CHECK(hipMemcpyAsync(g.x + n, up, n * 4, hipMemcpyHostToDevice, g.s));
    if (!launch_silu(g.x, g.x + n, (int)n, g.y, g.s)) return 0;
    RH_CHECK(hipMemcpyAsync(out, g.y, n * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    return 1;
}

__global__ void f16_kernel(const uint16_t *h, int n, float *out) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) out[i] = h2f(h[i]);
}
int rusty_hip_debug_f16(const uint16_t *h, uintptr_t n, float *out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !h || !out || n == 0) return 0;
    if (!ensure(&g.x, &g.x_cap, n) || !ensure(&g.y, &g.y_cap, n)) return 0;
    RH_CHECK(hipMemcpyAsync(g.x, h, n * 2, hipMemcpyHostToDevice, g.s));
    rh_launch(f16_kernel, dim3(256), dim3(256), 0, g.s, (const uint16_t *)g.x, (int)n, g.y);
    RH_LAUNCH_OK();
    RH_CHECK(hipMemcpyAsync(out, g.y, n * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    return 1;
}

int rusty_hip_debug_rope(float *q, float *k, uint32_t pos, uint32_t hd, uint32_t nh, uint32_t nkv,
                         const float *inv_freq, uint32_t neox) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !q || !k || !inv_freq || hd == 0 || hd % 2 != 0) return 0;
    size_t half = hd / 2, nq = (size_t)nh * hd, nk = (size_t)nkv * hd;
    std::vector<float> ct(half), stb(half);
    for (size_t i = 0; i < half; i++) {
        float ang = (float)pos * inv_freq[i];
        stb[i] = sinf(ang);
        ct[i] = cosf(ang);
    }
    // device: [q | k | cache_k (nk) | cache_v (1 float) | cos | sin]
    if (!ensure(&g.x, &g.x_cap, nq + 2 * nk + 2 * half + 4)) return 0;
    float *dq = g.x, *dk = dq + nq, *ck = dk + nk, *dcos = ck + nk, *dsin = dcos + half;
    RH_CHECK(hipMemcpyAsync(dq, q, nq * 4, hipMemcpyHostToDevice, g.s));
    RH_CHECK(hipMemcpyAsync(dk, k, nk * 4, hipMemcpyHostToDevice, g.s));
    RH_CHECK(hipMemcpyAsync(dcos, ct.data(), half * 4, hipMemcpyHostToDevice, g.s));
    RH_CHECK(hipMemcpyAsync(dsin, stb.data(), half * 4, hipMemcpyHostToDevice, g.s));
    RopeArgs A;
    memset(&A, 0, sizeof(A));
    A.q = dq;
    A.k = dk;
    A.v = dk;
    A.kcache = ck;
    A.vcache = ck;  // value copy writes are disabled by n_kv*vd = 0 below
    A.cos_t = dcos;
    A.sin_t = dsin;
    A.pos = 0;
    A.max_pos = 1;
    A.n_heads = (int)nh;
    A.n_kv = (int)nkv;
    A.hd = (int)hd;
    A.vd = 0;
    A.slots = 1;
    A.ring = 0;
    A.neox = (int)neox;
    rh_launch(rope_kv_kernel, dim3(64), dim3(256), 0, g.s, A);
    RH_LAUNCH_OK();
    RH_CHECK(hipMemcpyAsync(q, dq, nq * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipMemcpyAsync(k, ck, nk * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    return 1;
}

}  // extern "C"

// ===== resident decoder ====================================================================
namespace rh {

struct RLayer {
    DevW w[7];
    float *attn_norm = nullptr, *ffn_norm = nullptr;  // gpt-oss: ffn_norm is post_attn_norm
    float *bias[3] = {nullptr, nullptr, nullptr};
    float *k = nullptr, *v = nullptr;
    float *vt = nullptr;  // transposed V copy [n_kv*vd][vt_stride] (standard layers)
    // gpt-oss
    float *bo = nullptr, *sinks = nullptr;
    MoeDev moe{};
};

struct Resident {
    bool configured = false, ready = false;
    uint32_t n_layers = 0, dim = 0, n_heads = 0, n_kv = 0, hd = 0, vd = 0, hidden = 0, vocab = 0;
    // storage: KV slots per layer; max_pos: positions the decoder accepts
    // (rows of the RoPE table, the longest attention range).  They differ
    // only for a ring cache (gpt-oss with a sliding window: storage =
    // min(window, max_pos), slot = pos % storage, KVCache::storage_len_for /
    // slot_for_pos, src/model.rs:1450-1464).
    uint32_t storage = 0, max_pos = 0;
    bool ring = false;
    // KV cache elements in bf16 (KVCache::enable_bf16, src/model.rs:1406-1421)
    bool kv_bf16 = false;
    uint32_t neox = 0;
    uint32_t vt_stride = 0;  // positions per row of the transposed V copies (storage rounded up to 64)
    float eps = 1e-5f;
    std::vector<RLayer> L;
    float *x = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr;
    float *hid = nullptr, *tg = nullptr, *tu = nullptr, *logits = nullptr;
    XQ xq_dim{}, xq_attn{}, xq_hid{};
    DevW out_w;
    float *out_norm = nullptr, *cos_t = nullptr, *sin_t = nullptr;
    DevW embd;
    bool has_embd = false;
    StepState *st = nullptr;
    StepState *st_host = nullptr;  // pinned staging
    float *part = nullptr;
    int n_chunks = 1;
    float *ex = nullptr;  // exact-attention scratch
    int ex_cap = 0;
    uint32_t *sync = nullptr;  // streamed exact attention: epoch, ticket, timeouts, flags [n_kv][ex_cap/64]
    size_t sync_words = 0;
    float *am_v = nullptr;
    int32_t *am_i = nullptr;
    uint32_t *ticket = nullptr;
    int32_t *tokens = nullptr;   // device prompt / output tokens
    int32_t *out_idx = nullptr;
    uint32_t tok_cap = 0;
    int am_blocks = 256;
    // gpt-oss mode
    bool moe = false;
    uint32_t n_exp = 0, top_k = 0, window = 0;
    float rope_conc = 1.0f;
    float *moebuf = nullptr;
    // batched prefill, allocated on first use for pf_cap tokens per chunk
    uint32_t pf_cap = 0;
    float *px = nullptr, *pq = nullptr, *pk = nullptr, *pv = nullptr, *pattn = nullptr, *ptg = nullptr,
          *ptu = nullptr, *pex = nullptr;
    int8_t *pbq = nullptr;
    // batched gpt-oss prefill, on top of the above: normalized rows, the
    // linear K/V buffers of the ring layers, router and expert rows
    float *pxn = nullptr, *plk = nullptr, *plv = nullptr, *plog = nullptr, *pprob = nullptr, *pgate = nullptr,
          *pup = nullptr, *pproj = nullptr;
    int32_t *psel = nullptr;
    // the matrix-core expert product's per-expert pair lists, counts and
    // tile offsets (rusty_hip_set_expert_mfma)
    int32_t *plists = nullptr, *pcounts = nullptr, *ptile0 = nullptr;
    std::map<std::pair<int, uint32_t>, hipGraphExec_t> graphs;  // by (mode, penalty bits)
    std::vector<void *> allocs;
    std::vector<std::pair<const void *, DevW>> wown;  // weight copies owned by the decoder
};
static Resident R;

enum { MODE_DEVTOK = 1, MODE_LOGITS = 2, MODE_GREEDY = 4 };

static int r_alloc(void **p, size_t bytes) {
    RH_CHECK(hipMalloc(p, bytes));
    R.allocs.push_back(*p);
    return 1;
}

// The resident decoder's own device copy of a weight, freed only by the next
// configure: a tensor given twice (a tied output head) is copied once.
static int r_weight(const uint8_t *host, size_t len, int64_t rows, int64_t cols, int fmt, DevW *out) {
    if (!weight_shape_ok(host, len, rows, cols, fmt)) return 0;
    for (const auto &e : R.wown)
        if (e.first == (const void *)host && e.second.rows == rows && e.second.cols == cols && e.second.fmt == fmt) {
            *out = e.second;
            return 1;
        }
    DevW w;
    if (!upload_weight(host, rows, cols, fmt, 0, &w)) return 0;
    R.allocs.push_back((void *)w.p);
    R.wown.emplace_back((const void *)host, w);
    *out = w;
    return 1;
}

static void r_reset() {
    if (g.s) (void)hipStreamSynchronize(g.s);
    for (auto &kv : R.graphs) (void)hipGraphExecDestroy(kv.second);
    R.graphs.clear();
    for (void *p : R.allocs) (void)hipFree(p);
    R.allocs.clear();
    R.wown.clear();
    if (R.st_host) (void)hipHostFree(R.st_host);
    R.st_host = nullptr;
    R.L.clear();
    R.configured = R.ready = false;
    R.has_embd = false;
    R.tok_cap = 0;
    R.moe = false;
    R.kv_bf16 = false;
    R.n_exp = R.top_k = R.window = 0;
    R.rope_conc = 1.0f;
    R.moebuf = nullptr;
    R.pf_cap = 0;
    R.pxn = nullptr;  // with the other batched-prefill buffers, freed through allocs
}

static void r_invalidate_graphs() {
    if (!R.graphs.empty()) (void)hipStreamSynchronize(g.s);  // no exec may still be in flight
    for (auto &kv : R.graphs) (void)hipGraphExecDestroy(kv.second);
    R.graphs.clear();
}
void r_invalidate_graphs_extern() { r_invalidate_graphs(); }

// Whether every streamed attention launch since the last check finished its
// bounded waits.  A wait that ran out marked its launch in sync[2] and the
// launch ended with wrong values; the call that ran it must then report
// failure (return 0, like the Metal decoder's incomplete command buffer,
// metal_backend.m:1254-1257).  The whole flag block is cleared so the next
// launch starts from epoch 0 with no stale flags; the captured graphs read
// the epoch at run time and stay valid.  The stream must be idle.
static int r_stream_ok() {
    if (!R.sync) return 1;
    uint32_t mark = 0;
    RH_CHECK(hipMemcpy(&mark, R.sync + 2, 4, hipMemcpyDeviceToHost));
    if (mark == 0) return 1;
    if (debug_on()) fprintf(stderr, "[rusty_hip] streamed attention: a bounded wait ran out; results invalid\n");
    RH_CHECK(hipMemset(R.sync, 0, R.sync_words * 4));
    RH_CHECK(hipDeviceSynchronize());
    return 0;
}

static int dt_to_fmt(uint32_t dt) {
    switch (dt) {
    case 0: return 12;
    case 1: return 14;
    case 2: return 8;
    case 3: return 39;
    case 8: case 12: case 14: case 39: return (int)dt;
    default: return -1;
    }
}

// RMSNorm of the residual stream as a GEMV activation.
static ActSpec r_act_norm(const float *norm_w) {
    ActSpec a;
    memset(&a, 0, sizeof(a));
    a.mode = ACT_RMSNORM;
    a.x = R.x;
    a.norm_w = norm_w;
    a.eps = R.eps;
    a.xq = R.xq_dim;
    a.xn = R.xn;
    return a;
}

// V rows [slot][w] of slots slot0..slot0+n-1 into the tiled transposed copy
// (vt4_off layout, vt_stride slots per column).
__global__ void kv_transpose_kernel(const float *v, int w, int slot0, int n, float *vt, int vt_stride) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)n * w) return;
    const int t = (int)(i / w), j = (int)(i % w);
    vt[vt4_off(j, slot0 + t, vt_stride)] = v[(int64_t)(slot0 + t) * w + j];
}

// Split-K attention for this decoder: the mode switch, except with a bf16
// KV cache, which only the reference-order kernels read.
static bool r_fast() { return attn_fast_mode() && !R.kv_bf16; }

// bf16 V rows of slots slot0..slot0+n-1, widened, into the tiled f32 copy.
__global__ void kv_transpose16_kernel(const uint16_t *v, int w, int slot0, int n, float *vt, int vt_stride) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)n * w) return;
    const int t = (int)(i / w), j = (int)(i % w);
    vt[vt4_off(j, slot0 + t, vt_stride)] = bf16_to_f32(v[(int64_t)(slot0 + t) * w + j]);
}

// One token through the layer stack (and head / greedy by mode) on stream s.
static int r_enqueue_moe(int mode, float penalty, hipStream_t s);
// The wo rows the next launch computes, for the streamed attention's
// scores workgroups to load into each XCD's L2 (AttnExactArgs.pf): only for
// the launch shape that maps row groups to XCDs simply, a K-quant wo with one
// row per wave tile (K <= 4096) and the attention-normalisation prologue,
// whose persistent grid is a multiple of 8 workgroups taking four rows (one
// per wave) at a time.  RUSTY_HIP_WO_PREFETCH=0 turns it off.
static void wo_prefetch(const DevW &w, int K, const float *attn, int vd, AttnExactArgs &E) {
    static int on = -1;
    if (on < 0) {
        const char *e = getenv("RUSTY_HIP_WO_PREFETCH");
        on = (e && e[0] == '0') ? 0 : 1;
    }
    E.pf = nullptr;
    ActSpec a;
    memset(&a, 0, sizeof(a));
    a.mode = ACT_DEN;
    a.x = (float *)attn;
    a.group = vd;
    if (!on || kq_prologue_act(a, K) != KQ_ACT_DEN || K > 4096 || (w.fmt != 12 && w.fmt != 14)) return;
    const int grid = w.fmt == 12 ? persistent_grid(gemv_kq_kernel<12, false, 1, KQ_ACT_DEN>, w.rows, 4, GK_PRO)
                                 : persistent_grid(gemv_kq_kernel<14, false, 1, KQ_ACT_DEN>, w.rows, 4, GK_PRO);
    if (grid % 8 != 0) return;
    E.pf = w.p;
    E.pf_stride = w.stride;
    E.pf_rows = w.rows;
    E.pf_group_rows = 4;
}

static int r_enqueue(int mode, float penalty, hipStream_t s) {
    if (R.moe) return r_enqueue_moe(mode, penalty, s);
    const int dim = R.dim, qd = R.n_heads * R.hd, kd = R.n_kv * R.hd, vdim = R.n_kv * R.vd;
    const int attn_cols = R.n_heads * R.vd;
    if (mode & MODE_DEVTOK) {
        ProfScope ps("embed", s);
        rh_launch(embed_kernel, dim3((dim + 255) / 256), dim3(256), 0, s, R.embd.p, R.embd.stride,
                           R.embd.fmt, dim, R.st, 0, R.x);
        RH_LAUNCH_OK();
    }
    for (uint32_t l = 0; l < R.n_layers; l++) {
        RLayer &Ly = R.L[l];
        MatSpec qkv[3] = {{Ly.w[0], R.q, Ly.bias[0]}, {Ly.w[1], R.k, Ly.bias[1]}, {Ly.w[2], R.v, Ly.bias[2]}};
        if (!gemv_multi_act(qkv, 3, dim, EPI_STORE, r_act_norm(Ly.attn_norm), s)) return 0;
        RopeArgs r_rope;
        {
            RopeArgs A;
            memset(&A, 0, sizeof(A));
            A.q = R.q;
            A.k = R.k;
            A.v = R.v;
            A.kcache = Ly.k;
            A.vcache = Ly.v;
            A.vtcache = Ly.vt;
            A.vt_stride = (int32_t)R.vt_stride;
            A.cos_t = R.cos_t;
            A.sin_t = R.sin_t;
            A.st = R.st;
            A.max_pos = R.max_pos;
            A.n_heads = R.n_heads;
            A.n_kv = R.n_kv;
            A.hd = R.hd;
            A.vd = R.vd;
            A.slots = R.storage;
            A.ring = 0;
            A.neox = R.neox;
            A.kv_bf16 = R.kv_bf16 ? 1 : 0;
            r_rope = A;
            if (r_fast()) {
                int work = R.n_heads * (R.hd / 2) + R.n_kv * (R.hd / 2) + vdim;
                ProfScope ps("rope_kv", s);
                rh_launch(rope_kv_kernel, dim3((work + 255) / 256), dim3(256), 0, s, A);
                RH_LAUNCH_OK();
            }
        }
        ActSpec act_o = act_xq(attn_cols % 256 == 0 ? R.xq_attn : XQ{}, R.attn);
        act_o.xq = attn_cols % 256 == 0 ? R.xq_attn : XQ{};
        if (r_fast()) {
            AttnArgs A;
            memset(&A, 0, sizeof(A));
            A.q = R.q;
            A.k = Ly.k;
            A.v = Ly.v;
            A.sinks = nullptr;
            A.part = R.part;
            A.out = R.attn;
            A.xq = (attn_cols % 256 == 0) ? R.xq_attn : XQ{};
            A.st = R.st;
            A.n_heads = R.n_heads;
            A.n_kv = R.n_kv;
            A.kv_mul = R.n_heads / R.n_kv;
            A.hd = R.hd;
            A.vd = R.vd;
            A.key_stride = kd;
            A.value_stride = vdim;
            A.slot_count = R.storage;
            A.window = 0;
            A.n_chunks = R.n_chunks;
            A.scale = 1.0f / sqrtf((float)R.hd);
            if (!attn_launch(A, s)) return 0;
        } else {
            AttnExactArgs E;
            memset(&E, 0, sizeof(E));
            E.q = R.q;
            E.k = Ly.k;
            E.v = Ly.v;
            E.vt = Ly.vt;
            E.vt_stride = (int32_t)R.vt_stride;
            E.out = R.attn;
            E.st = R.st;
            E.n_heads = R.n_heads;
            E.n_kv = R.n_kv;
            E.kv_mul = R.n_heads / R.n_kv;
            E.hd = R.hd;
            E.vd = R.vd;
            E.key_stride = kd;
            E.value_stride = vdim;
            E.slot_count = R.storage;
            E.window = 0;
            E.cap = R.ex_cap;
            E.scale = 1.0f / sqrtf((float)R.hd);
            E.rope = r_rope;  // RoPE + KV store inside the scores launch
            E.fuse_rope = 1;
            E.kv_bf16 = R.kv_bf16 ? 1 : 0;
            E.start_t = R.st_host ? R.st_host->start_t : 0;  // the range's start as of this enqueue (a hint)
            wo_prefetch(Ly.w[3], attn_cols, R.attn, R.vd, E);
            const float *den = nullptr;
            if (!attn_exact_launch(E, R.ex, XQ{}, s, false, &den, R.sync)) return 0;
            act_o.mode = ACT_DEN;
            act_o.den = den;
            act_o.group = R.vd;
        }
        MatSpec mo = {Ly.w[3], R.x, nullptr};
        if (!gemv_multi_act(&mo, 1, attn_cols, EPI_ADD, act_o, s)) return 0;
        if (!gemv_swiglu_act(Ly.w[4], Ly.w[5], dim, r_act_norm(Ly.ffn_norm), R.hid, R.tg, R.tu, s)) return 0;
        ActSpec act_h;
        memset(&act_h, 0, sizeof(act_h));
        act_h.mode = ACT_QUANT;
        act_h.x = R.hid;
        act_h.xq = R.xq_hid;
        MatSpec md = {Ly.w[6], R.x, nullptr};
        if (!gemv_multi_act(&md, 1, R.hidden, EPI_ADD, act_h, s)) return 0;
    }
    (void)qd;
    if (mode & (MODE_LOGITS | MODE_GREEDY)) {
        MatSpec mh = {R.out_w, R.logits, nullptr};
        if (!gemv_multi_act(&mh, 1, dim, EPI_STORE, r_act_norm(R.out_norm), s)) return 0;
    }
    if (mode & MODE_GREEDY) {
        ArgmaxArgs A;
        memset(&A, 0, sizeof(A));
        A.logits = R.logits;
        A.n = R.vocab;
        A.penalty = penalty;
        A.st = R.st;
        A.part_v = R.am_v;
        A.part_i = R.am_i;
        A.ticket = R.ticket;
        A.out_tokens = R.tokens;
        A.out_index = R.out_idx;
        A.advance = 1;
        ProfScope ps("argmax_greedy", s);
        rh_launch(argmax_greedy_kernel, dim3(R.am_blocks), dim3(256), 0, s, A);
        RH_LAUNCH_OK();
    }
    return 1;
}

// One gpt-oss token (forward_gpt_oss_into, src/model.rs:6733-6908).
static int r_enqueue_moe(int mode, float penalty, hipStream_t s) {
    const int dim = R.dim, vdim = R.n_kv * R.vd, kd = R.n_kv * R.hd;
    const int attn_cols = R.n_heads * R.vd;
    if (mode & MODE_DEVTOK) {
        ProfScope ps("embed", s);
        rh_launch(embed_kernel, dim3((dim + 255) / 256), dim3(256), 0, s, R.embd.p, R.embd.stride, R.embd.fmt, dim,
                  R.st, 0, R.x);
        RH_LAUNCH_OK();
    }
    for (uint32_t l = 0; l < R.n_layers; l++) {
        RLayer &Ly = R.L[l];
        MatSpec qkv[3] = {{Ly.w[0], R.q, Ly.bias[0]}, {Ly.w[1], R.k, Ly.bias[1]}, {Ly.w[2], R.v, Ly.bias[2]}};
        if (!gemv_multi_act(qkv, 3, dim, EPI_STORE, r_act_norm(Ly.attn_norm), s)) return 0;
        // The exact path stores the current position's K/V inside its scores
        // launch, unless another position of the range shares its ring slot
        // (a full-range layer past the ring's length reads that slot as the
        // reference does after the store: the store must come first).
        const int window = (l % 2 == 0) ? (int)R.window : 0;
        const bool rope_in_scores = !attn_fast_mode() && (!R.ring || window > 0);
        RopeArgs r_rope;
        {
            RopeArgs A;
            memset(&A, 0, sizeof(A));
            A.q = R.q;
            A.k = R.k;
            A.v = R.v;
            A.kcache = Ly.k;
            A.vcache = Ly.v;
            A.cos_t = R.cos_t;
            A.sin_t = R.sin_t;
            A.st = R.st;
            A.max_pos = R.max_pos;
            A.n_heads = R.n_heads;
            A.n_kv = R.n_kv;
            A.hd = R.hd;
            A.vd = R.vd;
            A.slots = R.storage;
            A.ring = R.ring ? 1 : 0;  // KVCache::k_offset(pos) (src/model.rs:6778-6783)
            A.neox = 0;
            r_rope = A;
            if (!rope_in_scores) {
                int work = R.n_heads * (R.hd / 2) + R.n_kv * (R.hd / 2) + vdim;
                ProfScope ps("rope_kv", s);
                rh_launch(rope_kv_kernel, dim3((work + 255) / 256), dim3(256), 0, s, A);
                RH_LAUNCH_OK();
            }
        }
        // attention with sinks; even layers see the sliding window only
        // (attention_start_pos, src/model.rs:6788-6792)
        ActSpec act_o = act_xq(attn_cols % 256 == 0 ? R.xq_attn : XQ{}, R.attn);
        if (attn_fast_mode()) {
            AttnArgs A;
            memset(&A, 0, sizeof(A));
            A.q = R.q;
            A.k = Ly.k;
            A.v = Ly.v;
            A.sinks = Ly.sinks;
            A.part = R.part;
            A.out = R.attn;
            A.xq = (attn_cols % 256 == 0) ? R.xq_attn : XQ{};
            A.st = R.st;
            A.n_heads = R.n_heads;
            A.n_kv = R.n_kv;
            A.kv_mul = R.n_heads / R.n_kv;
            A.hd = R.hd;
            A.vd = R.vd;
            A.key_stride = kd;
            A.value_stride = vdim;
            A.slot_count = R.storage;
            A.window = window;
            A.n_chunks = R.n_chunks;
            A.scale = 1.0f / sqrtf((float)R.hd);
            if (!attn_launch(A, s)) return 0;
        } else {
            AttnExactArgs E;
            memset(&E, 0, sizeof(E));
            E.q = R.q;
            E.k = Ly.k;
            E.v = Ly.v;
            E.sinks = Ly.sinks;
            E.out = R.attn;
            E.st = R.st;
            E.n_heads = R.n_heads;
            E.n_kv = R.n_kv;
            E.kv_mul = R.n_heads / R.n_kv;
            E.hd = R.hd;
            E.vd = R.vd;
            E.key_stride = kd;
            E.value_stride = vdim;
            E.slot_count = R.storage;
            E.window = window;
            E.cap = R.ex_cap;
            E.scale = 1.0f / sqrtf((float)R.hd);
            E.rope = r_rope;  // RoPE + KV store inside the scores launch (or a rope_kv launch it makes)
            E.fuse_rope = rope_in_scores ? 1 : 0;
            const float *den = nullptr;
            if (!attn_exact_launch(E, R.ex, XQ{}, s, false, &den, R.sync)) return 0;
            act_o.mode = ACT_DEN;
            act_o.den = den;
            act_o.group = R.vd;
        }
        // x += wo attn + bo (src/model.rs:6837-6840)
        MatSpec mo = {Ly.w[3], R.x, Ly.bo};
        if (!gemv_multi_act(&mo, 1, attn_cols, EPI_ADD, act_o, s)) return 0;
        // xn2 = rms_norm(x, post_attn_norm); x += moe(xn2)
        if (!moe_ffn_enqueue(Ly.moe, R.xn, dim % 256 == 0 ? R.xq_dim : XQ{}, nullptr, R.x, R.moebuf, s, nullptr, nullptr,
                             R.x, Ly.ffn_norm, R.eps))
            return 0;
    }
    if (mode & (MODE_LOGITS | MODE_GREEDY)) {
        MatSpec mh = {R.out_w, R.logits, nullptr};
        if (!gemv_multi_act(&mh, 1, dim, EPI_STORE, r_act_norm(R.out_norm), s)) return 0;
    }
    if (mode & MODE_GREEDY) {
        ArgmaxArgs A;
        memset(&A, 0, sizeof(A));
        A.logits = R.logits;
        A.n = R.vocab;
        A.penalty = penalty;
        A.st = R.st;
        A.part_v = R.am_v;
        A.part_i = R.am_i;
        A.ticket = R.ticket;
        A.out_tokens = R.tokens;
        A.out_index = R.out_idx;
        A.advance = 1;
        ProfScope ps("argmax_greedy", s);
        rh_launch(argmax_greedy_kernel, dim3(R.am_blocks), dim3(256), 0, s, A);
        RH_LAUNCH_OK();
    }
    return 1;
}

static bool use_graphs() {
    if (g.prof.on) return false;
    const char *e = getenv("RUSTY_HIP_GRAPH");
    return !(e && strcmp(e, "0") == 0);
}

// Runs one token in `mode`, via a cached graph when allowed.  The penalty is
// baked into the greedy graph, so graphs are keyed by (mode, penalty bits).
// The token graph for (mode, penalty), captured on first use.
static int r_graph(int mode, float penalty, hipGraphExec_t *out) {
    uint32_t pb;
    memcpy(&pb, &penalty, 4);
    const auto key = std::make_pair(mode, pb);
    auto it = R.graphs.find(key);
    if (it == R.graphs.end()) {
        hipGraph_t graph;
        RH_CHECK(hipStreamBeginCapture(g.s, hipStreamCaptureModeThreadLocal));
        int ok = r_enqueue(mode, penalty, g.s);
        hipError_t e = hipStreamEndCapture(g.s, &graph);
        if (!ok || e != hipSuccess) {
            if (e == hipSuccess) (void)hipGraphDestroy(graph);
            return 0;
        }
        hipGraphExec_t exec;
        hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        RH_CHECK(ie);
        it = R.graphs.emplace(key, exec).first;
    }
    *out = it->second;
    return 1;
}

static int r_run(int mode, float penalty) {
    if (!use_graphs()) return r_enqueue(mode, penalty, g.s);
    hipGraphExec_t exec;
    if (!r_graph(mode, penalty, &exec)) return 0;
    RH_CHECK(hipGraphLaunch(exec, g.s));
    return 1;
}

// ---- batched prefill (forward_prefill_batch, src/model.rs:9917-10090) -----------
// A chunk of T prompt tokens goes through every layer together: each weight
// matrix is read once per chunk by the batched products on the matrix cores,
// while RMSNorm, bias, RoPE, the KV store and attention stay per token with
// the decode step's arithmetic.  The KV cache is linear (slot = position), so
// the chunk's K/V rows are all stored before any of its tokens attends; each
// token's range ends at its own position, which is the sequential order's
// result exactly.  Every value written is bit-identical to decoding the
// tokens one by one.
// Tokens per chunk: RUSTY_HIP_PREFILL_CHUNK (64..2048), else 512 (a sweep
// over 256/512/1024 on a 2048-token prompt put 512 first, by 2-4%).
static int pf_chunk() {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("RUSTY_HIP_PREFILL_CHUNK");
        v = e ? atoi(e) : 512;
        v = std::max(64, std::min(2048, v));
    }
    return v;
}

static bool r_prefill_enabled() {
    static int on = -1;
    if (on < 0) {
        const char *e = getenv("RUSTY_HIP_PREFILL");
        on = (e && (e[0] == '0' || e[0] == 'n' || e[0] == 'N' || e[0] == 'f' || e[0] == 'F')) ? 0 : 1;
    }
    return on == 1;
}

// standard_prefill_batchable (src/model.rs:9869-9887): a standard model whose
// seven projections are all K-quant, with K-quant-compatible widths.
static bool r_prefill_batchable() {
    if (!R.ready || R.moe || !R.has_embd) return false;
    if (R.dim % 256 != 0 || (R.n_heads * R.vd) % 256 != 0 || R.hidden % 256 != 0) return false;
    for (const RLayer &Ly : R.L)
        for (int i = 0; i < 7; i++)
            if (Ly.w[i].fmt != 12 && Ly.w[i].fmt != 14) return false;
    return true;
}

static int r_prefill_alloc() {
    if (R.pf_cap) return 1;
    const size_t C = (size_t)pf_chunk();
    const size_t qd = (size_t)R.n_heads * R.hd, kd = (size_t)R.n_kv * R.hd, vdim = (size_t)R.n_kv * R.vd;
    const size_t attn_cols = (size_t)R.n_heads * R.vd;
    const size_t kmax = std::max<size_t>(std::max<size_t>(R.dim, attn_cols), R.hidden);
    const size_t ex = exact_scratch_floats((int)R.n_kv, (int)(R.n_heads / R.n_kv), R.ex_cap);
    if (!r_alloc((void **)&R.px, C * R.dim * 4) || !r_alloc((void **)&R.pq, C * qd * 4) ||
        !r_alloc((void **)&R.pk, C * kd * 4) || !r_alloc((void **)&R.pv, C * vdim * 4) ||
        !r_alloc((void **)&R.pattn, C * attn_cols * 4) || !r_alloc((void **)&R.ptg, C * R.hidden * 4) ||
        !r_alloc((void **)&R.ptu, C * R.hidden * 4) || !r_alloc((void **)&R.pex, C * ex * 4) ||
        !r_alloc((void **)&R.pbq, batch_xq_bytes((int)C, (int)kmax)))
        return 0;
    R.pf_cap = (uint32_t)C;
    return 1;
}

static int r_rmsnorm_batch(const float *norm_w, int T, const BatchXq &b, hipStream_t s) {
    ProfScope ps("rmsnorm_q8k_batch", s);
    rh_launch(rmsnorm_q8k_batch_kernel, dim3((unsigned)T), dim3(256), R.dim * 4, s, (const float *)R.px,
              norm_w, R.eps, (int)R.dim, b.qs, b.dx, b.ldx);
    RH_LAUNCH_OK();
    return 1;
}

// T (<= pf_cap) tokens from the device array tok at positions pos0.. .
static int r_prefill_chunk(const int32_t *tok, int T, int pos0, hipStream_t s) {
    const int dim = R.dim, qd = R.n_heads * R.hd, kd = R.n_kv * R.hd, vdim = R.n_kv * R.vd;
    const int attn_cols = R.n_heads * R.vd, hid = R.hidden, kvm = R.n_heads / R.n_kv;
    if (T <= 0 || (uint32_t)T > R.pf_cap) return 0;
    {
        ProfScope ps("embed_batch", s);
        rh_launch(embed_batch_kernel, dim3((dim + 255) / 256, (unsigned)T), dim3(256), 0, s, R.embd.p, R.embd.stride,
                  R.embd.fmt, dim, tok, R.px);
        RH_LAUNCH_OK();
    }
    const BatchXq bd = batch_xq_at(R.pbq, T, dim), ba = batch_xq_at(R.pbq, T, attn_cols);
    const BatchXq bh = batch_xq_at(R.pbq, T, hid);
    const int cap = (pos0 + T + 63) / 64 * 64;
    for (uint32_t l = 0; l < R.n_layers; l++) {
        RLayer &Ly = R.L[l];
        if (!r_rmsnorm_batch(Ly.attn_norm, T, bd, s)) return 0;
        if (!gemm_kq_enqueue(Ly.w[0], bd, T, R.pq, qd, EPI_STORE, Ly.bias[0], s, "pf_gemm_q") ||
            !gemm_kq_enqueue(Ly.w[1], bd, T, R.pk, kd, EPI_STORE, Ly.bias[1], s, "pf_gemm_k") ||
            !gemm_kq_enqueue(Ly.w[2], bd, T, R.pv, vdim, EPI_STORE, Ly.bias[2], s, "pf_gemm_v"))
            return 0;
        {
            RopeArgs A;
            memset(&A, 0, sizeof(A));
            A.q = R.pq;
            A.k = R.pk;
            A.v = R.pv;
            A.kcache = Ly.k;
            A.vcache = Ly.v;
            A.vtcache = Ly.vt;
            A.vt_stride = (int32_t)R.vt_stride;
            A.cos_t = R.cos_t;
            A.sin_t = R.sin_t;
            A.st = nullptr;
            A.pos = pos0;
            A.max_pos = R.max_pos;
            A.n_heads = R.n_heads;
            A.n_kv = R.n_kv;
            A.hd = R.hd;
            A.vd = R.vd;
            A.slots = R.storage;
            A.ring = 0;
            A.neox = R.neox;
            A.kv_bf16 = R.kv_bf16 ? 1 : 0;
            A.q_tok = qd;
            A.k_tok = kd;
            A.v_tok = vdim;
            const int work = R.n_heads * (R.hd / 2) + R.n_kv * (R.hd / 2) + vdim;
            ProfScope ps("rope_kv_batch", s);
            rh_launch(rope_kv_kernel, dim3((work + 255) / 256, (unsigned)T), dim3(256), 0, s, A);
            RH_LAUNCH_OK();
        }
        {
            AttnExactArgs E;
            memset(&E, 0, sizeof(E));
            E.q = R.pq;
            E.k = Ly.k;
            E.v = Ly.v;
            E.vt = Ly.vt;
            E.vt_stride = (int32_t)R.vt_stride;
            E.out = R.pattn;
            E.n_heads = R.n_heads;
            E.n_kv = R.n_kv;
            E.kv_mul = kvm;
            E.hd = R.hd;
            E.vd = R.vd;
            E.key_stride = kd;
            E.value_stride = vdim;
            E.slot_count = R.storage;
            E.start_t = 0;
            E.window = 0;
            E.cap = cap;
            E.scale = 1.0f / sqrtf((float)R.hd);
            E.n_tok = T;
            E.pos0 = pos0;
            E.q_tok = qd;
            E.kv_bf16 = R.kv_bf16 ? 1 : 0;
            E.o_tok = attn_cols;
            const float *den = nullptr;
            if (!attn_exact_launch(E, R.pex, XQ{}, s, false, &den)) return 0;
            ProfScope ps("attn_finish_batch", s);
            rh_launch(attn_finish_q8k_batch_kernel, dim3(attn_cols / 256, (unsigned)T), dim3(256), 0, s,
                      (const float *)R.pattn, den, (int64_t)exact_scratch_floats(R.n_kv, kvm, cap), (int)R.vd,
                      attn_cols, ba.qs, ba.dx, ba.ldx);
            RH_LAUNCH_OK();
        }
        if (!gemm_kq_enqueue(Ly.w[3], ba, T, R.px, dim, EPI_ADD, nullptr, s, "pf_gemm_o")) return 0;
        if (!r_rmsnorm_batch(Ly.ffn_norm, T, bd, s)) return 0;
        if (!gemm_kq_enqueue(Ly.w[4], bd, T, R.ptg, hid, EPI_STORE, nullptr, s, "pf_gemm_gate_up") ||
            !gemm_kq_enqueue(Ly.w[5], bd, T, R.ptu, hid, EPI_STORE, nullptr, s, "pf_gemm_gate_up"))
            return 0;
        {
            ProfScope ps("silu_mul_batch", s);
            rh_launch(silu_mul_q8k_batch_kernel, dim3(hid / 256, (unsigned)T), dim3(256), 0, s, (const float *)R.ptg,
                      (const float *)R.ptu, hid, bh.qs, bh.dx, bh.ldx);
            RH_LAUNCH_OK();
        }
        if (!gemm_kq_enqueue(Ly.w[6], bh, T, R.px, dim, EPI_ADD, nullptr, s,
                             Ly.w[6].fmt == 12 ? "pf_gemm_down_q4k" : "pf_gemm_down_q6k"))
            return 0;
    }
    return 1;
}

// ---- batched gpt-oss prefill (forward_prefill_gpt_oss token by token,
// src/model.rs:10286) ----------------------------------------------------------
// The gpt-oss resident decoder batches when its attention projections and
// router are Q8_0, its experts MXFP4 and its KV f32.
static bool r_prefill_moe_batchable() {
    if (!R.ready || !R.moe || !R.has_embd || R.kv_bf16) return false;
    const int dim = (int)R.dim, attn_cols = (int)(R.n_heads * R.vd);
    if (dim % 32 != 0 || attn_cols % 256 != 0 || !cat_of(8, dim) || !cat_of(8, attn_cols)) return false;
    for (const RLayer &Ly : R.L) {
        for (int i = 0; i < 4; i++)
            if (Ly.w[i].fmt != 8) return false;
        const MoeDev &M = Ly.moe;
        if (M.router.fmt != 8 || M.gate.fmt != 39 || M.up.fmt != 39 || M.down.fmt != 39) return false;
        if (M.dim != dim || M.hidden % 32 != 0 || M.k < 1 || M.k > 8 || M.n_exp > 64) return false;
    }
    return true;
}

static int r_prefill_moe_alloc() {
    if (R.pxn) return 1;
    if (!r_prefill_alloc()) return 0;
    const size_t C = R.pf_cap, k = R.top_k, kd = (size_t)R.n_kv * R.hd, vdim = (size_t)R.n_kv * R.vd;
    const size_t hid = R.L.empty() ? 0 : (size_t)R.L[0].moe.hidden, rows = R.storage + C;
    if (!r_alloc((void **)&R.plk, rows * kd * 4) || !r_alloc((void **)&R.plv, rows * vdim * 4) ||
        !r_alloc((void **)&R.plog, C * 64 * 4) || !r_alloc((void **)&R.psel, C * k * 4) ||
        !r_alloc((void **)&R.pprob, C * k * 4) || !r_alloc((void **)&R.pgate, C * k * hid * 4) ||
        !r_alloc((void **)&R.pup, C * k * hid * 4) || !r_alloc((void **)&R.pproj, C * k * R.dim * 4) ||
        !r_alloc((void **)&R.pxn, C * R.dim * 4) || !r_alloc((void **)&R.plists, (size_t)64 * MXE_MAX_PAIRS * 4) ||
        !r_alloc((void **)&R.pcounts, 64 * 4) || !r_alloc((void **)&R.ptile0, 65 * 4))
        return 0;
    return 1;
}

// The expert product of the batched gpt-oss prefill: the reference's serial
// row sums (gemv_mxfp4_experts_kernel, bit-exact; the default) or, when
// rusty_hip_set_expert_mfma(1) chose it, the matrix cores (the pair lists
// first, then gemm_mxfp4_experts_mfma_kernel).  lists/counts/tile0: the list
// buffers; with lists_ready the lists of this sel are already built.
static int g_expert_mfma = -1;
static bool expert_mfma_on() {
    if (g_expert_mfma < 0) {
        const char *e = getenv("RUSTY_HIP_EXPERT_MFMA");
        g_expert_mfma = (e && e[0] == '1') ? 1 : 0;
    }
    return g_expert_mfma == 1;
}
static int experts_enqueue(MxExpArgs A, int n_mats, bool mfma, int32_t *lists, int32_t *counts, int32_t *tile0,
                           bool lists_ready, const char *name, hipStream_t s) {
    if (A.n_exp < 1 || A.n_exp > 64 || A.K % 32 != 0 || A.n_pairs <= 0 || A.rows <= 0 || n_mats < 1 || n_mats > 2)
        return 0;
    if (!mfma) {
        if (A.n_pairs > MXE_MAX_PAIRS * A.k) return 0;
        ProfScope ps(name, s);
        rh_launch(gemv_mxfp4_experts_kernel, dim3((unsigned)((A.rows + 63) / 64), (unsigned)A.n_exp, (unsigned)n_mats),
                  dim3(256), 0, s, A);
        RH_LAUNCH_OK();
        return 1;
    }
    // the activation rows are read as 16-byte pieces
    if (A.ldx % 4 != 0 || ((uintptr_t)A.x & 15) != 0 || A.row_stride % 16 != 0) return 0;
    if (!lists_ready) {
        ProfScope ps("moe_expert_lists", s);
        rh_launch(moe_expert_lists_kernel, dim3(1), dim3(256), 0, s, A.sel, A.n_pairs, A.n_exp, MXE_MAX_PAIRS, lists,
                  counts, tile0);
        RH_LAUNCH_OK();
    }
    // at most ceil(n_pairs / 32) + n_exp pair tiles in all
    const unsigned tiles = (unsigned)((A.n_pairs + MXM_PAIRS - 1) / MXM_PAIRS + A.n_exp);
    ProfScope ps(name, s);
    rh_launch(gemm_mxfp4_experts_mfma_kernel, dim3((unsigned)((A.rows + MXM_ROWS - 1) / MXM_ROWS), tiles,
                                                   (unsigned)n_mats),
              dim3(256), 0, s, A, (const int32_t *)lists, (const int32_t *)counts, (const int32_t *)tile0,
              (int)MXE_MAX_PAIRS);
    RH_LAUNCH_OK();
    return 1;
}

// y[t][r] (=, or += with EPI_ADD) Q8_0 row r of W times token t (+ bias):
// f32 activations x [T][K] or the batched Q8_K in bq, as cat_of picks for K.
static int q80_batch_enqueue(const DevW &W, int rows, int K, int T, const float *x, const BatchXq *bq,
                             const float *bias, float *y, int ldy, int epi, const char *name, hipStream_t s) {
    if (W.fmt != 8 || T <= 0) return 0;
    Q80BatchArgs A;
    memset(&A, 0, sizeof(A));
    A.w = W.p;
    A.row_stride = W.stride;
    A.rows = rows;
    A.K = K;
    A.T = T;
    A.epi = epi;
    A.bias = bias;
    A.y = y;
    A.ldy = ldy;
    const int cat = cat_of(8, K);
    ProfScope ps(name, s);
    const dim3 rg((unsigned)((rows + 31) / 32));
    if (cat == CAT_F32) {
        if (!x || K % 4 != 0) return 0;
        A.x = x;
        if (K <= 4096)
            rh_launch((gemv_q8_0_batch_kernel<true, 4>), dim3(rg.x, (unsigned)((T + 3) / 4)), dim3(256),
                      (size_t)4 * K * 4, s, A);
        else
            rh_launch((gemv_q8_0_batch_kernel<true, 1>), dim3(rg.x, (unsigned)T), dim3(256), (size_t)K * 4, s, A);
    } else if (cat == CAT_Q8I) {
        if (!bq) return 0;
        A.qs = bq->qs;
        A.dx = bq->dx;
        A.ldx = bq->ldx;
        if (K <= 8192)
            rh_launch((gemv_q8_0_batch_kernel<false, 8>), dim3(rg.x, (unsigned)((T + 7) / 8)), dim3(256),
                      (size_t)8 * K + 8 * (K / 256) * 4, s, A);
        else
            rh_launch((gemv_q8_0_batch_kernel<false, 2>), dim3(rg.x, (unsigned)((T + 1) / 2)), dim3(256),
                      (size_t)2 * K + 2 * (K / 256) * 4, s, A);
    } else {
        return 0;
    }
    RH_LAUNCH_OK();
    return 1;
}

// RMSNorm of the chunk's rows into R.pxn (f32), plus their Q8_K in b when
// the width takes the integer Q8_0 path.
static int r_norm_batch_moe(const float *norm_w, int T, const BatchXq &b, hipStream_t s) {
    const int dim = (int)R.dim;
    {
        ProfScope ps("rmsnorm_batch", s);
        rh_launch(rmsnorm_f32_batch_kernel, dim3((unsigned)((dim + 255) / 256), (unsigned)T), dim3(256),
                  (size_t)dim * 4, s, (const float *)R.px, norm_w, R.eps, dim, R.pxn);
        RH_LAUNCH_OK();
    }
    if (cat_of(8, dim) == CAT_Q8I && !quantize_batch_enqueue(R.pxn, dim, T, dim, b, s)) return 0;
    return 1;
}

static int kv_ring_copy(RLayer &Ly, int p0, int n, int off, int to_ring, hipStream_t s) {
    if (n <= 0) return 1;
    const int kd = (int)(R.n_kv * R.hd), vdim = (int)(R.n_kv * R.vd);
    ProfScope ps("kv_ring_copy", s);
    rh_launch(kv_ring_copy_kernel, dim3((unsigned)((std::max(kd, vdim) + 255) / 256), (unsigned)n, 2), dim3(256), 0, s,
              Ly.k, Ly.v, R.plk, R.plv, kd, vdim, p0, (int)R.storage, off, to_ring);
    RH_LAUNCH_OK();
    return 1;
}

// T (<= pf_cap) tokens of a gpt-oss model at positions pos0.. .  Each layer:
// RMSNorm, q/k/v (+ bias), RoPE with the K/V rows stored into a linear buffer
// that also holds the ring's rows of the S - 1 positions before the chunk,
// exact attention with sinks (window on even layers) where each token reads
// the ring as it stood at its own step, the chunk's last S rows written back
// to the ring, wo (+ bias, residual), RMSNorm, router, top-k, the experts'
// gate/up, SwiGLU, down, and the slot-ordered combine into the residual.
static int r_prefill_chunk_moe(const int32_t *tok, int T, int pos0, hipStream_t s) {
    const int dim = (int)R.dim, qd = (int)(R.n_heads * R.hd), kd = (int)(R.n_kv * R.hd), vdim = (int)(R.n_kv * R.vd);
    const int attn_cols = (int)(R.n_heads * R.vd), kvm = (int)(R.n_heads / R.n_kv), S = (int)R.storage;
    if (T <= 0 || (uint32_t)T > R.pf_cap || T > MXE_MAX_PAIRS) return 0;
    const int P0 = std::max(0, pos0 - S + 1), npre = pos0 - P0;
    {
        ProfScope ps("embed_batch", s);
        rh_launch(embed_batch_kernel, dim3((dim + 255) / 256, (unsigned)T), dim3(256), 0, s, R.embd.p, R.embd.stride,
                  R.embd.fmt, dim, tok, R.px);
        RH_LAUNCH_OK();
    }
    const BatchXq bd = batch_xq_at(R.pbq, T, dim), ba = batch_xq_at(R.pbq, T, attn_cols);
    const int cap = (pos0 + T + 63) / 64 * 64;
    const int last0 = std::max(pos0, pos0 + T - S);  // the chunk's positions the ring keeps
    for (uint32_t l = 0; l < R.n_layers; l++) {
        RLayer &Ly = R.L[l];
        const MoeDev &M = Ly.moe;
        if (!r_norm_batch_moe(Ly.attn_norm, T, bd, s)) return 0;
        if (!q80_batch_enqueue(Ly.w[0], qd, dim, T, R.pxn, &bd, Ly.bias[0], R.pq, qd, EPI_STORE, "pf_q80_q", s) ||
            !q80_batch_enqueue(Ly.w[1], kd, dim, T, R.pxn, &bd, Ly.bias[1], R.pk, kd, EPI_STORE, "pf_q80_k", s) ||
            !q80_batch_enqueue(Ly.w[2], vdim, dim, T, R.pxn, &bd, Ly.bias[2], R.pv, vdim, EPI_STORE, "pf_q80_v", s))
            return 0;
        if (!kv_ring_copy(Ly, P0, npre, 0, 0, s)) return 0;
        {
            RopeArgs A;
            memset(&A, 0, sizeof(A));
            A.q = R.pq;
            A.k = R.pk;
            A.v = R.pv;
            A.kcache = R.plk;
            A.vcache = R.plv;
            A.cos_t = R.cos_t;
            A.sin_t = R.sin_t;
            A.pos = pos0;
            A.max_pos = R.max_pos;
            A.n_heads = R.n_heads;
            A.n_kv = R.n_kv;
            A.hd = R.hd;
            A.vd = R.vd;
            A.slots = S;
            A.ring = 0;
            A.slot_off = P0;  // row = pos - P0 of the linear buffer
            A.neox = 0;
            A.q_tok = qd;
            A.k_tok = kd;
            A.v_tok = vdim;
            const int work = R.n_heads * (R.hd / 2) + R.n_kv * (R.hd / 2) + vdim;
            ProfScope ps("rope_kv_batch", s);
            rh_launch(rope_kv_kernel, dim3((work + 255) / 256, (unsigned)T), dim3(256), 0, s, A);
            RH_LAUNCH_OK();
        }
        {
            AttnExactArgs E;
            memset(&E, 0, sizeof(E));
            E.q = R.pq;
            E.k = R.plk;
            E.v = R.plv;
            E.sinks = Ly.sinks;
            E.out = R.pattn;
            E.n_heads = R.n_heads;
            E.n_kv = R.n_kv;
            E.kv_mul = kvm;
            E.hd = R.hd;
            E.vd = R.vd;
            E.key_stride = kd;
            E.value_stride = vdim;
            E.slot_count = S;
            E.start_t = 0;
            E.window = (l % 2 == 0) ? (int)R.window : 0;  // attention_start_pos, src/model.rs:6788-6792
            E.cap = cap;
            E.scale = 1.0f / sqrtf((float)R.hd);
            E.n_tok = T;
            E.pos0 = pos0;
            E.q_tok = qd;
            E.o_tok = attn_cols;
            E.lin = 1;
            E.lin_pos0 = P0;
            const float *den = nullptr;
            if (!attn_exact_launch(E, R.pex, XQ{}, s, false, &den)) return 0;
            ProfScope ps("attn_finish_batch", s);
            rh_launch(attn_finish_q8k_batch_kernel, dim3(attn_cols / 256, (unsigned)T), dim3(256), 0, s,
                      (const float *)R.pattn, den, (int64_t)exact_scratch_floats(R.n_kv, kvm, cap), (int)R.vd,
                      attn_cols, ba.qs, ba.dx, ba.ldx);
            RH_LAUNCH_OK();
        }
        if (!kv_ring_copy(Ly, last0, pos0 + T - last0, last0 - P0, 1, s)) return 0;
        // x += wo attn + bo (src/model.rs:6837-6840)
        if (!q80_batch_enqueue(Ly.w[3], dim, attn_cols, T, nullptr, &ba, Ly.bo, R.px, dim, EPI_ADD, "pf_q80_o", s))
            return 0;
        // xn2 = rms_norm(x, post_attn_norm); x += moe(xn2) (src/model.rs:6846-6898)
        if (!r_norm_batch_moe(Ly.ffn_norm, T, bd, s)) return 0;
        const int k = M.k, hid = M.hidden, np = T * k;
        const bool mfma = expert_mfma_on();
        if (!q80_batch_enqueue(M.router, M.n_exp, dim, T, R.pxn, &bd, M.router_bias, R.plog, 64, EPI_STORE,
                               "pf_router", s))
            return 0;
        {
            ProfScope ps("moe_topk_batch", s);
            rh_launch(moe_topk_batch_kernel, dim3((unsigned)T), dim3(64), 0, s, (const float *)R.plog, 64, M.n_exp, k,
                      R.psel, R.pprob);
            RH_LAUNCH_OK();
        }
        {
            MxExpArgs A;
            memset(&A, 0, sizeof(A));
            A.w[0] = M.gate.p;
            A.w[1] = M.up.p;
            A.y[0] = R.pgate;
            A.y[1] = R.pup;
            A.row_stride = M.gate.stride;
            A.exp_stride = (int64_t)hid * M.gate.stride;
            A.rows = hid;
            A.K = dim;
            A.n_pairs = np;
            A.k = k;
            A.x = R.pxn;
            A.ldx = dim;
            A.ldy = hid;
            A.x_pair = 0;
            A.sel = R.psel;
            A.n_exp = M.n_exp;
            if (M.up.stride != M.gate.stride) return 0;
            if (!experts_enqueue(A, 2, mfma, R.plists, R.pcounts, R.ptile0, false, "pf_mxfp4_gate_up", s)) return 0;
        }
        {
            ProfScope ps("moe_swiglu_batch", s);
            rh_launch(moe_swiglu_kernel, dim3((unsigned)((hid + 255) / 256), (unsigned)np), dim3(256), 0, s, R.pgate,
                      (const float *)R.pup, hid, np, (const int32_t *)R.psel, M.gb, M.gb_stride, M.ub, M.ub_stride);
            RH_LAUNCH_OK();
        }
        {
            MxExpArgs A;
            memset(&A, 0, sizeof(A));
            A.w[0] = M.down.p;
            A.y[0] = R.pproj;
            A.row_stride = M.down.stride;
            A.exp_stride = (int64_t)dim * M.down.stride;
            A.rows = dim;
            A.K = hid;
            A.n_pairs = np;
            A.k = k;
            A.x = R.pgate;
            A.ldx = hid;
            A.ldy = dim;
            A.x_pair = 1;
            A.sel = R.psel;
            A.n_exp = M.n_exp;
            if (!experts_enqueue(A, 1, mfma, R.plists, R.pcounts, R.ptile0, true, "pf_mxfp4_down", s)) return 0;
        }
        {
            ProfScope ps("moe_combine_batch", s);
            rh_launch(moe_combine_batch_kernel, dim3((unsigned)((dim + 255) / 256), (unsigned)T), dim3(256), 0, s,
                      (const float *)R.pproj, dim, k, (const int32_t *)R.psel, (const float *)R.pprob, M.db,
                      M.db_stride, R.px);
            RH_LAUNCH_OK();
        }
    }
    return 1;
}

// n tokens already in R.tokens[0..n) at positions pos0.. in chunks.
static int r_prefill_tokens(int n, int pos0) {
    if (R.moe) {
        if (!r_prefill_moe_alloc()) return 0;
        const int cap = std::min<int>((int)R.pf_cap, MXE_MAX_PAIRS);  // the experts' pair lists hold one chunk
        for (int c = 0; c < n; c += cap)
            if (!r_prefill_chunk_moe(R.tokens + c, std::min<int>(cap, n - c), pos0 + c, g.s)) return 0;
        return 1;
    }
    if (!r_prefill_alloc()) return 0;
    for (int c = 0; c < n; c += (int)R.pf_cap)
        if (!r_prefill_chunk(R.tokens + c, std::min<int>((int)R.pf_cap, n - c), pos0 + c, g.s)) return 0;
    return 1;
}

static int r_ensure_tokens(uint32_t need) {
    if (R.tok_cap >= need) return 1;
    need = std::max(need, std::min<uint32_t>(R.max_pos + 1, 8192));
    if (!r_alloc((void **)&R.tokens, (size_t)need * 4)) return 0;
    R.tok_cap = need;
    r_invalidate_graphs();  // the greedy graph records the token pointer
    return 1;
}

static int r_set_state(int pos, int start_t, int token, bool reset_recent) {
    StepState *h = R.st_host;
    RH_CHECK(hipStreamSynchronize(g.s));  // staging buffer reuse
    RH_CHECK(hipMemcpy(h, R.st, sizeof(StepState), hipMemcpyDeviceToHost));
    h->pos = pos;
    h->start_t = start_t;
    h->token = token;
    if (reset_recent) h->n_recent = 0;
    RH_CHECK(hipMemcpyAsync(R.st, h, sizeof(StepState), hipMemcpyHostToDevice, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    return 1;
}

}  // namespace rh

extern "C" {

}  // extern "C"

// Resident buffers for a model shape (shared by both configure calls).
// storage_len KV slots per layer, max_pos positions (max_pos > storage_len
// only for a ring cache).
static int r_setup(uint32_t n_layers, uint32_t dim, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                   uint32_t value_dim, uint32_t hidden_dim, uint32_t vocab, uint32_t storage_len, uint32_t max_pos,
                   float eps, uint32_t neox) {
    r_reset();
    R.n_layers = n_layers;
    R.dim = dim;
    R.n_heads = n_heads;
    R.n_kv = n_kv_heads;
    R.hd = head_dim;
    R.vd = value_dim;
    R.hidden = hidden_dim;
    R.vocab = vocab;
    R.storage = storage_len;
    R.max_pos = max_pos;
    R.ring = max_pos > storage_len;
    R.eps = eps;
    R.neox = neox;
    R.L.resize(n_layers);
    size_t qd = (size_t)n_heads * head_dim, kd = (size_t)n_kv_heads * head_dim, vdim = (size_t)n_kv_heads * value_dim;
    size_t attn_cols = (size_t)n_heads * value_dim;
    if (!r_alloc((void **)&R.x, dim * 4) || !r_alloc((void **)&R.xn, dim * 4) || !r_alloc((void **)&R.q, qd * 4) ||
        !r_alloc((void **)&R.k, kd * 4) || !r_alloc((void **)&R.v, vdim * 4) ||
        !r_alloc((void **)&R.attn, attn_cols * 4) || !r_alloc((void **)&R.hid, hidden_dim * 4) ||
        !r_alloc((void **)&R.tg, hidden_dim * 4) || !r_alloc((void **)&R.tu, hidden_dim * 4) ||
        !r_alloc((void **)&R.logits, (size_t)vocab * 4))
        return 0;
    XQ *xqs[3] = {&R.xq_dim, &R.xq_attn, &R.xq_hid};
    size_t ns[3] = {dim, attn_cols, hidden_dim};
    for (int i = 0; i < 3; i++) {
        size_t nb = (ns[i] + 255) / 256;
        if (!r_alloc((void **)&xqs[i]->qs, nb * 256) || !r_alloc((void **)&xqs[i]->d, nb * 4) ||
            !r_alloc((void **)&xqs[i]->bsums, nb * 16) || !r_alloc((void **)&xqs[i]->sums16, nb * 32))
            return 0;
    }
    R.n_chunks = attn_chunks((int)n_kv_heads, (int)max_pos);
    if (!r_alloc((void **)&R.part, (size_t)n_kv_heads * R.n_chunks * (n_heads / n_kv_heads) * att_pstride((int)value_dim) * 4))
        return 0;
    R.ex_cap = (int)((max_pos + 63) / 64 * 64);  // a range is at most max_pos positions
    if (!r_alloc((void **)&R.ex, exact_scratch_floats((int)n_kv_heads, (int)(n_heads / n_kv_heads), R.ex_cap) * 4)) return 0;
    const size_t sync_words = 3 + (size_t)n_kv_heads * (R.ex_cap / 64);
    if (!r_alloc((void **)&R.sync, sync_words * 4)) return 0;
    RH_CHECK(hipMemset(R.sync, 0, sync_words * 4));
    R.sync_words = sync_words;
    R.am_blocks = std::min<int>(256, (int)((vocab + 255) / 256));
    if (!r_alloc((void **)&R.am_v, R.am_blocks * 4) || !r_alloc((void **)&R.am_i, R.am_blocks * 4) ||
        !r_alloc((void **)&R.ticket, 64) || !r_alloc((void **)&R.st, sizeof(StepState)) ||
        !r_alloc((void **)&R.out_idx, 64))
        return 0;
    RH_CHECK(hipMemset(R.ticket, 0, 64));
    RH_CHECK(hipMemset(R.st, 0, sizeof(StepState)));
    RH_CHECK(hipMemset(R.out_idx, 0, 64));
    RH_CHECK(hipHostMalloc((void **)&R.st_host, sizeof(StepState), hipHostMallocDefault));
    R.configured = true;
    return 1;
}

extern "C" {

int rusty_hip_resident_configure(uint32_t n_layers, uint32_t dim, uint32_t n_heads, uint32_t n_kv_heads,
                                 uint32_t head_dim, uint32_t value_dim, uint32_t hidden_dim, uint32_t vocab,
                                 uint32_t storage_len, float eps, uint32_t neox) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked()) return 0;
    if (n_layers == 0 || n_layers > 512 || n_kv_heads == 0 || n_heads % n_kv_heads != 0) return 0;
    if (head_dim == 0 || head_dim > 256 || value_dim == 0 || value_dim > 256) return 0;
    if (dim % 256 != 0 || hidden_dim % 256 != 0 || storage_len == 0 || vocab == 0) return 0;
    if (!attn_supported((int)head_dim, (int)value_dim, (int)(n_heads / n_kv_heads))) return 0;
    return r_setup(n_layers, dim, n_heads, n_kv_heads, head_dim, value_dim, hidden_dim, vocab, storage_len,
                   storage_len, eps, neox);
}

int rusty_hip_resident_configure_moe(uint32_t n_layers, uint32_t dim, uint32_t n_heads, uint32_t n_kv_heads,
                                     uint32_t head_dim, uint32_t hidden_dim, uint32_t n_experts, uint32_t top_k,
                                     uint32_t vocab, uint32_t storage_len, uint32_t sliding_window, float eps,
                                     float rope_concentration) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked()) return 0;
    if (n_layers == 0 || n_layers > 512 || n_kv_heads == 0 || n_heads % n_kv_heads != 0) return 0;
    if (head_dim == 0 || head_dim > 256 || head_dim % 2 != 0) return 0;
    // f32-activation paths: dims in whole 32-blocks, within the LDS staging
    if (dim % 32 != 0 || hidden_dim % 32 != 0 || dim > 12288 || hidden_dim > 12288) return 0;
    if (storage_len == 0 || vocab == 0 || n_experts == 0 || n_experts > 64 || top_k == 0 || top_k > 8 ||
        top_k > n_experts)
        return 0;
    if (!attn_supported((int)head_dim, (int)head_dim, (int)(n_heads / n_kv_heads))) return 0;
    // storage_len is the cache's max_len; with a window the cache is a ring
    // of min(window, max_len) slots (KVCache::with_sliding_window,
    // src/model.rs:1363-1385, storage_len_for :1450-1455)
    const uint32_t slots = sliding_window > 0 ? std::min(sliding_window, storage_len) : storage_len;
    if (!r_setup(n_layers, dim, n_heads, n_kv_heads, head_dim, head_dim, hidden_dim, vocab, slots, storage_len, eps,
                 0))
        return 0;
    R.moe = true;
    R.n_exp = n_experts;
    R.top_k = top_k;
    R.window = sliding_window;
    R.rope_conc = rope_concentration;
    if (!r_alloc((void **)&R.moebuf, (moe_scratch_floats((int)n_experts, (int)top_k, (int)dim, (int)hidden_dim) + 8) * 4))
        return 0;
    return 1;
}

int rusty_hip_resident_set_moe_layer(uint32_t l, const RustyMoeLayerDesc *d) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!R.configured || !R.moe || !d || l >= R.n_layers) return 0;
    RLayer &Ly = R.L[l];
    const uint32_t qd = R.n_heads * R.hd, kd = R.n_kv * R.hd, vdim = R.n_kv * R.vd, ac = R.n_heads * R.vd;
    const uint32_t rows[4] = {qd, kd, vdim, R.dim}, cols[4] = {R.dim, R.dim, R.dim, ac};
    for (int i = 0; i < 4; i++) {
        const int fmt = dt_to_fmt(d->w_dt[i]);
        if (!d->w[i] || fmt < 0 || !cat_of(fmt, (int)cols[i])) return 0;
        if (!r_weight(d->w[i], d->w_len[i], rows[i], cols[i], fmt, &Ly.w[i])) return 0;
    }
    auto upload = [&](const float *h, size_t n, float **dst) {
        if (!h) return 0;
        if (!r_alloc((void **)dst, n * 4)) return 0;
        RH_CHECK(hipMemcpy(*dst, h, n * 4, hipMemcpyHostToDevice));
        return 1;
    };
    if (!upload(d->bq, qd, &Ly.bias[0]) || !upload(d->bk, kd, &Ly.bias[1]) || !upload(d->bv, vdim, &Ly.bias[2]) ||
        !upload(d->bo, R.dim, &Ly.bo) || !upload(d->sinks, R.n_heads, &Ly.sinks) ||
        !upload(d->attn_norm, R.dim, &Ly.attn_norm) || !upload(d->post_attn_norm, R.dim, &Ly.ffn_norm))
        return 0;
    MoeDev &M = Ly.moe;
    memset(&M, 0, sizeof(M));
    M.n_exp = (int)R.n_exp;
    M.k = (int)R.top_k;
    M.dim = (int)R.dim;
    M.hidden = (int)R.hidden;
    const int rfmt = dt_to_fmt(d->router_dt), efmt = dt_to_fmt(d->exps_dt);
    if (rfmt < 0 || efmt < 0 || !d->router) return 0;
    if (!r_weight(d->router, d->router_len, R.n_exp, R.dim, rfmt, &M.router)) return 0;
    const uint32_t erows[3] = {R.n_exp * R.hidden, R.n_exp * R.hidden, R.n_exp * R.dim};
    const uint32_t ecols[3] = {R.dim, R.dim, R.hidden};
    DevW *ew[3] = {&M.gate, &M.up, &M.down};
    for (int i = 0; i < 3; i++)
        if (!d->exps[i] || !r_weight(d->exps[i], d->exps_len[i], erows[i], ecols[i], efmt, ew[i])) return 0;
    float *rb = nullptr, *gb = nullptr, *ub = nullptr, *db = nullptr;
    if (d->router_bias && !upload(d->router_bias, R.n_exp, &rb)) return 0;
    if (d->exps_bias[0] && !upload(d->exps_bias[0], (size_t)R.n_exp * R.hidden, &gb)) return 0;
    if (d->exps_bias[1] && !upload(d->exps_bias[1], (size_t)R.n_exp * R.hidden, &ub)) return 0;
    if (d->exps_bias[2] && !upload(d->exps_bias[2], (size_t)R.n_exp * R.dim, &db)) return 0;
    M.router_bias = rb;
    M.gb = gb;
    M.ub = ub;
    M.db = db;
    M.gb_stride = M.ub_stride = (int)R.hidden;
    M.db_stride = (int)R.dim;
    size_t kdim = (size_t)R.n_kv * R.hd;
    if (!r_alloc((void **)&Ly.k, (size_t)R.storage * kdim * 4) || !r_alloc((void **)&Ly.v, (size_t)R.storage * vdim * 4))
        return 0;
    RH_CHECK(hipMemset(Ly.k, 0, (size_t)R.storage * kdim * 4));
    RH_CHECK(hipMemset(Ly.v, 0, (size_t)R.storage * vdim * 4));
    r_invalidate_graphs();
    return 1;
}

int rusty_hip_resident_set_layer(uint32_t l, const RustyResidentLayerDesc *d) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!R.configured || !d || l >= R.n_layers) return 0;
    RLayer &Ly = R.L[l];
    uint32_t cols[7] = {R.dim, R.dim, R.dim, R.n_heads * R.vd, R.dim, R.dim, R.hidden};
    uint32_t want_rows[7] = {R.n_heads * R.hd, R.n_kv * R.hd, R.n_kv * R.vd, R.dim, R.hidden, R.hidden, R.dim};
    for (int i = 0; i < 7; i++) {
        int fmt = dt_to_fmt(d->w_dt[i]);
        if (!d->w[i] || fmt < 0 || d->w_rows[i] != want_rows[i] || !cat_of(fmt, (int)cols[i])) return 0;
        if (!r_weight(d->w[i], d->w_len[i], d->w_rows[i], cols[i], fmt, &Ly.w[i])) return 0;
    }
    if (!d->attn_norm || !d->ffn_norm) return 0;
    if (!r_alloc((void **)&Ly.attn_norm, R.dim * 4) || !r_alloc((void **)&Ly.ffn_norm, R.dim * 4)) return 0;
    RH_CHECK(hipMemcpy(Ly.attn_norm, d->attn_norm, R.dim * 4, hipMemcpyHostToDevice));
    RH_CHECK(hipMemcpy(Ly.ffn_norm, d->ffn_norm, R.dim * 4, hipMemcpyHostToDevice));
    const float *bs[3] = {d->bq, d->bk, d->bv};
    uint32_t bl[3] = {d->bq_len, d->bk_len, d->bv_len};
    for (int i = 0; i < 3; i++) {
        Ly.bias[i] = nullptr;
        if (bs[i] && bl[i]) {
            if (bl[i] != want_rows[i]) return 0;
            if (!r_alloc((void **)&Ly.bias[i], bl[i] * 4)) return 0;
            RH_CHECK(hipMemcpy(Ly.bias[i], bs[i], bl[i] * 4, hipMemcpyHostToDevice));
        }
    }
    size_t kd = (size_t)R.n_kv * R.hd, vdim = (size_t)R.n_kv * R.vd;
    if (!r_alloc((void **)&Ly.k, (size_t)R.storage * kd * 4) || !r_alloc((void **)&Ly.v, (size_t)R.storage * vdim * 4))
        return 0;
    RH_CHECK(hipMemset(Ly.k, 0, (size_t)R.storage * kd * 4));
    RH_CHECK(hipMemset(Ly.v, 0, (size_t)R.storage * vdim * 4));
    R.vt_stride = (R.storage + 63) / 64 * 64;
    if (!r_alloc((void **)&Ly.vt, (size_t)R.vt_stride * vdim * 4)) return 0;
    RH_CHECK(hipMemset(Ly.vt, 0, (size_t)R.vt_stride * vdim * 4));
    r_invalidate_graphs();
    return 1;
}

int rusty_hip_resident_set_output(const float *output_norm, const uint8_t *output_w, uintptr_t output_w_len,
                                  uint32_t output_rows, uint32_t output_dt, const float *inv_freq,
                                  uint32_t inv_freq_len) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!R.configured || !output_norm || !output_w || !inv_freq || output_rows != R.vocab) return 0;
    if (inv_freq_len < R.hd / 2) return 0;
    int fmt = dt_to_fmt(output_dt);
    if (fmt < 0 || !cat_of(fmt, (int)R.dim)) return 0;
    if (!r_weight(output_w, output_w_len, output_rows, R.dim, fmt, &R.out_w)) return 0;
    if (!r_alloc((void **)&R.out_norm, R.dim * 4)) return 0;
    RH_CHECK(hipMemcpy(R.out_norm, output_norm, R.dim * 4, hipMemcpyHostToDevice));
    // RoPE table: the reference's angle (float)pos * inv_freq[i] and libm
    // sinf/cosf (apply_rope_qk, src/model.rs:5574-5575).
    size_t half = R.hd / 2;
    std::vector<float> ct((size_t)R.max_pos * half), stb((size_t)R.max_pos * half);
    for (size_t p = 0; p < R.max_pos; p++)
        for (size_t i = 0; i < half; i++) {
            float ang = (float)p * inv_freq[i];
            // gpt-oss scales both by the YaRN concentration (apply_rope_gpt_oss,
            // src/model.rs:6617-6619); 1.0 leaves them unchanged
            stb[p * half + i] = R.moe ? sinf(ang) * R.rope_conc : sinf(ang);
            ct[p * half + i] = R.moe ? cosf(ang) * R.rope_conc : cosf(ang);
        }
    if (!r_alloc((void **)&R.cos_t, ct.size() * 4) || !r_alloc((void **)&R.sin_t, stb.size() * 4)) return 0;
    RH_CHECK(hipMemcpy(R.cos_t, ct.data(), ct.size() * 4, hipMemcpyHostToDevice));
    RH_CHECK(hipMemcpy(R.sin_t, stb.data(), stb.size() * 4, hipMemcpyHostToDevice));
    for (uint32_t l = 0; l < R.n_layers; l++)
        if (!R.L[l].k) return 0;
    r_invalidate_graphs();
    R.ready = true;
    return 1;
}

int rusty_hip_resident_set_embedding(const uint8_t *embd, uintptr_t embd_len, uint32_t t) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!R.configured || !embd) return 0;
    int fmt = (int)t;
    if (row_bytes_of(fmt, R.dim) <= 0) return 0;
    if (!r_weight(embd, embd_len, R.vocab, R.dim, fmt, &R.embd)) return 0;
    R.has_embd = true;
    r_invalidate_graphs();
    return 1;
}

int rusty_hip_resident_decode(const float *x_embed, uint32_t pos, uint32_t start_t, int want_logits,
                              float *logits_out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!R.ready || !x_embed || pos >= R.max_pos) return 0;
    if (want_logits && !logits_out) return 0;
    // forward_gpt_oss_into has no start_t: its full layers scan from 0
    if (R.moe) start_t = 0;
    if (!r_set_state((int)pos, (int)start_t, 0, false)) return 0;
    RH_CHECK(hipMemcpyAsync(R.x, x_embed, R.dim * 4, hipMemcpyHostToDevice, g.s));
    if (!r_run(want_logits ? MODE_LOGITS : 0, 1.0f)) return 0;
    if (want_logits) RH_CHECK(hipMemcpyAsync(logits_out, R.logits, (size_t)R.vocab * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    prof_drain();
    return r_stream_ok();
}

int rusty_hip_resident_generate(const int32_t *prompt, uint32_t n_prompt, uint32_t start_pos, uint32_t n_gen,
                                float penalty, int32_t *out_tokens, float *logits_out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!R.ready || !R.has_embd || !prompt || n_prompt == 0 || (n_gen > 0 && !out_tokens)) return 0;
    if ((uint64_t)start_pos + n_prompt + n_gen > (uint64_t)R.max_pos + 1) return 0;
    for (uint32_t i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || (uint32_t)prompt[i] >= R.vocab) return 0;
    if (!r_ensure_tokens(std::max(n_prompt, n_gen) + 1)) return 0;
    RH_CHECK(hipMemcpy(R.tokens, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice));
    if (!r_set_state((int)start_pos, 0, prompt[0], true)) return 0;
    // prefill_prompt_tokens (src/runtime.rs:3368-3420): every prompt token but
    // the last in batched chunks when the model allows it, then the last one
    // through the decode step for its logits.
    const bool batched =
        n_prompt > 2 && r_prefill_enabled() && (r_prefill_batchable() || r_prefill_moe_batchable());
    if (batched && !r_prefill_tokens((int)n_prompt - 1, (int)start_pos)) return 0;
    // recent window = last <= 64 prompt tokens (recent_token_tail, src/runtime.rs:508-512)
    uint32_t tail = n_prompt > 64 ? n_prompt - 64 : 0;
    for (uint32_t i = 0; i < n_prompt; i++) {
        if (batched && i < tail && i + 1 < n_prompt) continue;  // no state change, no decode step
        rh_launch(set_step_kernel, dim3(1), dim3(64), 0, g.s, R.st, R.tokens, (int)i, (int)(start_pos + i),
                           i >= tail ? 1 : 0);
        RH_LAUNCH_OK();
        if (i + 1 < n_prompt && !batched) {
            if (!r_run(MODE_DEVTOK, 1.0f)) return 0;
        }
    }
    RH_CHECK(hipMemsetAsync(R.out_idx, 0, 4, g.s));
    if (n_gen == 0) {
        if (!r_run(MODE_DEVTOK | MODE_LOGITS, 1.0f)) return 0;
    } else {
        // The prompt copy in R.tokens is consumed; generated tokens overwrite it.
        for (uint32_t i = 0; i < n_gen; i++)
            if (!r_run(MODE_DEVTOK | MODE_GREEDY, penalty)) return 0;
        RH_CHECK(hipMemcpyAsync(out_tokens, R.tokens, (size_t)n_gen * 4, hipMemcpyDeviceToHost, g.s));
    }
    if (logits_out) RH_CHECK(hipMemcpyAsync(logits_out, R.logits, (size_t)R.vocab * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    prof_drain();
    return r_stream_ok();
}

int rusty_hip_resident_prefill(const int32_t *tokens, uint32_t n_tokens, uint32_t start_pos) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!tokens || n_tokens == 0 || !(r_prefill_batchable() || r_prefill_moe_batchable())) return 0;
    // positions: the cache's slots, or the decoder's range for a ring cache
    if ((uint64_t)start_pos + n_tokens > (uint64_t)(R.moe ? R.max_pos : R.storage)) return 0;
    for (uint32_t i = 0; i < n_tokens; i++)
        if (tokens[i] < 0 || (uint32_t)tokens[i] >= R.vocab) return 0;
    if (!r_ensure_tokens(n_tokens + 1)) return 0;
    RH_CHECK(hipMemcpy(R.tokens, tokens, (size_t)n_tokens * 4, hipMemcpyHostToDevice));
    if (!r_prefill_tokens((int)n_tokens, (int)start_pos)) return 0;
    RH_CHECK(hipStreamSynchronize(g.s));
    prof_drain();
    return 1;
}

int rusty_hip_set_expert_mfma(int on) {
    std::lock_guard<std::mutex> lk(g.mu);
    const int prev = expert_mfma_on() ? 1 : 0;
    g_expert_mfma = on ? 1 : 0;
    return prev;
}

int rusty_hip_mxfp4_experts(const uint8_t *w, int64_t row_stride, int64_t exp_stride, uint32_t n_exp, uint32_t rows,
                            uint32_t cols, const float *x, int64_t ldx, int x_per_pair, uint32_t top_k,
                            const int32_t *sel, uint32_t n_pairs, float *y, int64_t ldy, int mfma) {
    std::lock_guard<std::mutex> lk(g.mu);
    // n_pairs <= 1024: an expert's pair list holds at most that many
    if (!init_locked() || !w || !x || !sel || !y || n_exp < 1 || n_exp > 64 || rows < 1 || cols < 32 ||
        cols % 32 != 0 || top_k < 1 || top_k > 8 || n_pairs < 1 || n_pairs > (uint32_t)MXE_MAX_PAIRS ||
        row_stride < (int64_t)cols / 32 * 17 || row_stride % 16 != 0 || exp_stride < (int64_t)rows * row_stride ||
        ldy < (int64_t)rows || ldx < (int64_t)cols)
        return 0;
    static int32_t *lists[64] = {};  // per device: pair lists, counts, tile offsets
    if (g.dev < 0 || g.dev >= 64) return 0;
    int32_t *&L = lists[g.dev];
    if (mfma && !L && hipMalloc((void **)&L, ((size_t)64 * MXE_MAX_PAIRS + 64 + 65) * 4) != hipSuccess) {
        L = nullptr;
        return 0;
    }
    MxExpArgs A;
    memset(&A, 0, sizeof(A));
    A.w[0] = w;
    A.y[0] = y;
    A.row_stride = row_stride;
    A.exp_stride = exp_stride;
    A.rows = (int32_t)rows;
    A.K = (int32_t)cols;
    A.n_pairs = (int32_t)n_pairs;
    A.k = (int32_t)top_k;
    A.x = x;
    A.ldx = ldx;
    A.ldy = ldy;
    A.x_pair = x_per_pair ? 1 : 0;
    A.sel = sel;
    A.n_exp = (int32_t)n_exp;
    RH_CHECK(hipDeviceSynchronize());  // the caller's writes of w, x and sel are complete
    int32_t *lp = L, *cp = L ? L + (size_t)64 * MXE_MAX_PAIRS : nullptr, *tp = cp ? cp + 64 : nullptr;
    if (!experts_enqueue(A, 1, mfma != 0, lp, cp, tp, false, mfma ? "mxfp4_experts_mfma" : "mxfp4_experts", g.s))
        return 0;
    RH_CHECK(hipStreamSynchronize(g.s));
    prof_drain();
    return 1;
}

int rusty_hip_resident_time_decode(uint32_t n_tokens, float penalty, double *ms) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!R.ready || !R.has_embd || !ms) return 0;
    if (R.tok_cap < n_tokens + 1) {
        uint32_t need = std::max<uint32_t>(n_tokens + 1, std::min<uint32_t>(R.max_pos + 1, 8192));
        if (!r_alloc((void **)&R.tokens, (size_t)need * 4)) return 0;
        R.tok_cap = need;
        r_invalidate_graphs();
    }
    RH_CHECK(hipStreamSynchronize(g.s));
    RH_CHECK(hipMemcpy(R.st_host, R.st, sizeof(StepState), hipMemcpyDeviceToHost));
    if ((uint64_t)R.st_host->pos + n_tokens > R.max_pos) return 0;
    RH_CHECK(hipMemsetAsync(R.out_idx, 0, 4, g.s));
    // make sure the graph exists before timing
    if (use_graphs()) {
        // capture only (no launch): the replays below are timed
        hipGraphExec_t exec;
        if (!r_graph(MODE_DEVTOK | MODE_GREEDY, penalty, &exec)) return 0;
    }
    hipEvent_t a, b;
    RH_CHECK(hipEventCreate(&a));
    RH_CHECK(hipEventCreate(&b));
    RH_CHECK(hipEventRecord(a, g.s));
    for (uint32_t i = 0; i < n_tokens; i++)
        if (!r_run(MODE_DEVTOK | MODE_GREEDY, penalty)) return 0;
    RH_CHECK(hipEventRecord(b, g.s));
    RH_CHECK(hipEventSynchronize(b));
    float t = 0.0f;
    RH_CHECK(hipEventElapsedTime(&t, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    *ms = t;
    prof_drain();
    return r_stream_ok();
}

// Test hook for the streamed attention's timeout path: marks the next
// streamed launch (the epoch it will read) as timed out, as a bounded wait
// that ran out would, so every wait of that launch returns at once and the
// launch ends normally with invalid results.  0 when no streamed launch is
// configured.
int rusty_hip_debug_stream_mark(void) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!R.ready || !R.sync) return 0;
    RH_CHECK(hipStreamSynchronize(g.s));
    uint32_t ep = 0;
    RH_CHECK(hipMemcpy(&ep, R.sync, 4, hipMemcpyDeviceToHost));
    const uint32_t mark = ep + 1;
    RH_CHECK(hipMemcpy(R.sync + 2, &mark, 4, hipMemcpyHostToDevice));
    return 1;
}

// KV elements are f32, or bf16 (uint16) after rusty_hip_resident_enable_bf16.
int rusty_hip_resident_kv_read(uint32_t l, uint32_t which, uint32_t slot0, uint32_t n_slots, float *host_out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!R.configured || l >= R.n_layers || !host_out || (uint64_t)slot0 + n_slots > R.storage) return 0;
    const size_t w = which ? (size_t)R.n_kv * R.vd : (size_t)R.n_kv * R.hd, es = R.kv_bf16 ? 2 : 4;
    const char *src = (const char *)(which ? R.L[l].v : R.L[l].k);
    if (!src) return 0;
    RH_CHECK(hipStreamSynchronize(g.s));
    RH_CHECK(hipMemcpy(host_out, src + (size_t)slot0 * w * es, (size_t)n_slots * w * es, hipMemcpyDeviceToHost));
    return 1;
}

int rusty_hip_resident_kv_write(uint32_t l, uint32_t which, uint32_t slot0, uint32_t n_slots, const float *host_in) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!R.configured || l >= R.n_layers || !host_in || (uint64_t)slot0 + n_slots > R.storage) return 0;
    const size_t w = which ? (size_t)R.n_kv * R.vd : (size_t)R.n_kv * R.hd, es = R.kv_bf16 ? 2 : 4;
    char *dst = (char *)(which ? R.L[l].v : R.L[l].k);
    if (!dst) return 0;
    RH_CHECK(hipStreamSynchronize(g.s));
    RH_CHECK(hipMemcpy(dst + (size_t)slot0 * w * es, host_in, (size_t)n_slots * w * es, hipMemcpyHostToDevice));
    if (which && R.L[l].vt && n_slots > 0) {
        if (R.kv_bf16)
            rh_launch(kv_transpose16_kernel, dim3((n_slots * w + 255) / 256), dim3(256), 0, g.s, (const uint16_t *)dst,
                      (int)w, (int)slot0, (int)n_slots, R.L[l].vt, (int)R.vt_stride);
        else
            rh_launch(kv_transpose_kernel, dim3((n_slots * w + 255) / 256), dim3(256), 0, g.s, (const float *)dst,
                      (int)w, (int)slot0, (int)n_slots, R.L[l].vt, (int)R.vt_stride);
        RH_LAUNCH_OK();
        RH_CHECK(hipStreamSynchronize(g.s));
    }
    return 1;
}

// KVCache::enable_bf16 (src/model.rs:1406-1421) for the resident decoder.
int rusty_hip_resident_enable_bf16(int on) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!R.configured || R.moe) return 0;  // the reference keeps bf16 KV to the standard architecture
    const bool want = on != 0;
    if (want != R.kv_bf16) {
        R.kv_bf16 = want;
        // a fresh cache of the new element type (the buffers hold f32 either way)
        RH_CHECK(hipStreamSynchronize(g.s));
        const size_t kd = (size_t)R.n_kv * R.hd, vdim = (size_t)R.n_kv * R.vd;
        for (RLayer &Ly : R.L) {
            if (Ly.k) RH_CHECK(hipMemset(Ly.k, 0, (size_t)R.storage * kd * 4));
            if (Ly.v) RH_CHECK(hipMemset(Ly.v, 0, (size_t)R.storage * vdim * 4));
            if (Ly.vt) RH_CHECK(hipMemset(Ly.vt, 0, (size_t)R.vt_stride * vdim * 4));
        }
        r_invalidate_graphs();
    }
    return 1;
}

int rusty_hip_debug_greedy(const float *logits, uintptr_t n, const int32_t *recent, uint32_t n_recent, float penalty,
                           int32_t *token) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !logits || n == 0 || !token || n_recent > 64) return 0;
    // scratch: logits | partials | state
    size_t blocks = std::min<size_t>(256, (n + 255) / 256);
    size_t need = n + 2 * blocks + sizeof(StepState) / 4 + 64;
    if (!ensure(&g.y, &g.y_cap, need)) return 0;
    float *dl = g.y;
    float *pv = dl + n;
    int32_t *pi = (int32_t *)(pv + blocks);
    StepState *st = (StepState *)(pi + blocks);
    uint32_t *ticket = (uint32_t *)(st + 1);
    StepState hs;
    memset(&hs, 0, sizeof(hs));
    hs.n_recent = (int)n_recent;
    for (uint32_t i = 0; i < n_recent; i++) hs.recent[i] = recent[i];
    RH_CHECK(hipMemcpyAsync(dl, logits, n * 4, hipMemcpyHostToDevice, g.s));
    RH_CHECK(hipMemcpyAsync(st, &hs, sizeof(hs), hipMemcpyHostToDevice, g.s));
    RH_CHECK(hipMemsetAsync(ticket, 0, 4, g.s));
    ArgmaxArgs A;
    memset(&A, 0, sizeof(A));
    A.logits = dl;
    A.n = (int)n;
    A.penalty = penalty;
    A.st = st;
    A.part_v = pv;
    A.part_i = pi;
    A.ticket = ticket;
    A.advance = 1;
    rh_launch(argmax_greedy_kernel, dim3((unsigned)blocks), dim3(256), 0, g.s, A);
    RH_LAUNCH_OK();
    RH_CHECK(hipMemcpyAsync(&hs, st, sizeof(hs), hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    *token = hs.token;
    return 1;
}

// matvec_kquant_batch_into (src/simd.rs:3417-3435): one K-quant matrix
// against a row-major batch of activations, out row-major [T][rows].  Byte
// lengths as the other exports; inputs must hold a whole number of
// cols-wide rows and cols must be a multiple of 256, as the reference gates.
int rusty_hip_kquant_matvec_batch(uint32_t kind, const uint8_t *w, uintptr_t w_len, uintptr_t rows, uintptr_t cols,
                                  const float *inputs, uintptr_t inputs_len, float *out, uintptr_t out_len) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !w || !inputs || !out || rows == 0 || cols == 0 || cols % 256 != 0) return 0;
    const int fmt = dt_to_fmt(kind);
    if (fmt != 12 && fmt != 14) return 0;
    if (inputs_len == 0 || inputs_len % (cols * 4) != 0) return 0;
    const size_t T = inputs_len / (cols * 4);
    if (T > (1u << 20) || out_len < T * rows * 4) return 0;
    DevW W;
    if (!get_weight(w, w_len, (int64_t)rows, (int64_t)cols, fmt, &W)) return 0;
    if (!ensure(&g.bx, &g.bx_cap, T * cols) || !ensure(&g.by, &g.by_cap, T * rows) ||
        !ensure(&g.bq, &g.bq_cap, batch_xq_bytes((int)T, (int)cols)))
        return 0;
    const BatchXq b = batch_xq_at(g.bq, (int)T, (int)cols);
    RH_CHECK(hipMemcpyAsync(g.bx, inputs, T * cols * 4, hipMemcpyHostToDevice, g.s));
    if (!quantize_batch_enqueue(g.bx, (int)cols, (int)T, (int)cols, b, g.s)) return 0;
    if (!gemm_kq_enqueue(W, b, (int)T, g.by, (int)rows, EPI_STORE, nullptr, g.s)) return 0;
    RH_CHECK(hipMemcpyAsync(out, g.by, T * rows * 4, hipMemcpyDeviceToHost, g.s));
    RH_CHECK(hipStreamSynchronize(g.s));
    prof_drain();
    return 1;
}


// ---- kernel sweep (bench.py --sweep) ------------------------------------------------
// Both exports time kernels on device-resident inputs: nothing crosses PCIe
// inside the loop, and the inputs rotate over `copies` device copies so a
// launch streams from HBM rather than from the caches a previous launch
// filled.  Kernel durations are recorded by the profile (its families) when
// profiling is on; the result of the last launch is returned.

// iters GEMV launches y = W x (x quantized to Q8_K once, on the device, where
// the reference quantizes it).
int rusty_hip_bench_matvec(uint32_t t, const uint8_t *w, uintptr_t wl, const float *x, uintptr_t rows, uintptr_t cols,
                           uint32_t copies, uint32_t iters, float *out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !w || !x || !out || rows == 0 || cols == 0 || copies == 0 || copies > 64 || iters == 0)
        return 0;
    const int fmt = dt_to_fmt(t);
    const int cat = fmt > 0 ? cat_of(fmt, (int)cols) : 0;
    if (!cat) return 0;
    DevW W;
    if (!get_weight(w, wl, (int64_t)rows, (int64_t)cols, fmt, &W)) return 0;
    const size_t bytes = (size_t)W.rows * W.stride;
    std::vector<uint8_t *> cp(copies, nullptr);
    cp[0] = (uint8_t *)W.p;
    int ok = 1;
    for (uint32_t i = 1; i < copies && ok; i++) {
        if (hipMalloc((void **)&cp[i], bytes) != hipSuccess ||
            hipMemcpyAsync(cp[i], W.p, bytes, hipMemcpyDeviceToDevice, g.s) != hipSuccess)
            ok = 0;
    }
    if (ok) ok = stage_x(x, cols) && ensure(&g.y, &g.y_cap, rows);
    ActSpec act = act_xq(XQ{}, g.x);  // g.x as staged above
    if (ok && (cat == CAT_KQ || cat == CAT_Q8I)) {
        ok = ensure_xq(&g.xq, &g.xq_cap, cols) && launch_quant(g.x, (int)cols, g.xq, g.s);
        act = act_xq(g.xq, g.x);
    }
    for (uint32_t i = 0; i < iters && ok; i++) {
        DevW Wi = W;
        Wi.p = cp[i % copies];
        MatSpec m = {Wi, g.y, nullptr};
        ok = gemv_cat(&m, 1, (int)cols, EPI_STORE, act, g.s);
    }
    if (ok) ok = hipMemcpyAsync(out, g.y, rows * 4, hipMemcpyDeviceToHost, g.s) == hipSuccess;
    (void)hipStreamSynchronize(g.s);
    for (uint32_t i = 1; i < copies; i++)
        if (cp[i]) (void)hipFree(cp[i]);
    prof_drain();
    return ok;
}

// Pseudo-normal fill (sum of four hashed uniforms, variance 1) for the
// attention sweep's K, V and q.
__global__ void bench_fill_kernel(float *p, size_t n, uint32_t seed) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t h = (uint32_t)i * 0x9E3779B1u ^ (seed + 0x85EBCA77u * (uint32_t)(k + 1)) ^ (uint32_t)(i >> 32);
            h ^= h >> 16;
            h *= 0x7FEB352Du;
            h ^= h >> 15;
            h *= 0x846CA68Bu;
            h ^= h >> 16;
            acc += (float)(h >> 8) * (1.0f / 16777216.0f);
        }
        p[i] = (acc - 2.0f) * 1.7320508f;
    }
}

// iters decode-attention launches: heads query heads over kv_mul-way grouped
// K/V of ctx positions (linear slots), head_dim = value_dim, scale
// 1/sqrt(head_dim); mode 0 = the exact kernels, 1 = split-K.  out receives
// the last launch's heads*head_dim outputs.
int rusty_hip_bench_attention(uint32_t heads, uint32_t kv_mul, uint32_t head_dim, uint32_t ctx, uint32_t copies,
                              uint32_t iters, uint32_t seed, int mode, float *out) {
    std::lock_guard<std::mutex> lk(g.mu);
    if (!init_locked() || !out || heads == 0 || kv_mul == 0 || heads % kv_mul != 0 || ctx == 0 || copies == 0 ||
        copies > 256 || iters == 0 || !attn_supported((int)head_dim, (int)head_dim, (int)kv_mul))
        return 0;
    const int n_kv = (int)(heads / kv_mul), hd = (int)head_dim;
    const size_t per = (size_t)ctx * n_kv * hd;  // floats of K (and of V) per copy
    const size_t qn = (size_t)heads * hd;
    float *kv = nullptr;
    if (hipMalloc((void **)&kv, (2 * per * copies + qn) * sizeof(float)) != hipSuccess) return 0;
    float *q = kv + 2 * per * copies;
    int ok = 1;
    rh_launch(bench_fill_kernel, dim3(2048), dim3(256), 0, g.s, kv, 2 * per * copies + qn, seed);
    if (hipGetLastError() != hipSuccess) ok = 0;
    if (ok) ok = ensure(&g.y, &g.y_cap, qn);
    if (ok && mode == 1) {
        const int chunks = attn_chunks(n_kv, (int)ctx);
        ok = ensure(&g.part, &g.part_cap, (size_t)n_kv * chunks * kv_mul * att_pstride((int)head_dim));
    }
    const int cap = (int)((ctx + 63) / 64 * 64);
    if (ok && mode == 0) ok = ensure(&g.ex, &g.ex_cap, exact_scratch_floats(n_kv, (int)kv_mul, cap));
    for (uint32_t i = 0; i < iters && ok; i++) {
        const float *k = kv + 2 * per * (i % copies), *v = k + per;
        if (mode == 1) {
            AttnArgs A;
            memset(&A, 0, sizeof(A));
            A.q = q;
            A.k = k;
            A.v = v;
            A.part = g.part;
            A.out = g.y;
            A.n_heads = (int)heads;
            A.n_kv = n_kv;
            A.kv_mul = (int)kv_mul;
            A.hd = A.vd = hd;
            A.key_stride = A.value_stride = (int64_t)n_kv * hd;
            A.slot_count = (int)ctx;
            A.start_t = 0;
            A.end_t = (int)ctx - 1;
            A.n_chunks = attn_chunks(n_kv, (int)ctx);
            A.scale = 1.0f / sqrtf((float)hd);
            ok = attn_launch(A, g.s);
        } else {
            AttnExactArgs E;
            memset(&E, 0, sizeof(E));
            E.q = q;
            E.k = k;
            E.v = v;
            E.out = g.y;
            E.n_heads = (int)heads;
            E.n_kv = n_kv;
            E.kv_mul = (int)kv_mul;
            E.hd = E.vd = hd;
            E.key_stride = E.value_stride = (int64_t)n_kv * hd;
            E.slot_count = (int)ctx;
            E.start_t = 0;
            E.end_t = (int)ctx - 1;
            E.cap = cap;
            E.scale = 1.0f / sqrtf((float)hd);
            ok = attn_exact_launch(E, g.ex, XQ{}, g.s);
        }
    }
    if (ok) ok = hipMemcpyAsync(out, g.y, qn * 4, hipMemcpyDeviceToHost, g.s) == hipSuccess;
    (void)hipStreamSynchronize(g.s);
    (void)hipFree(kv);
    prof_drain();
    return ok;
}

// ---- GGUF on-disk path (src/gguf.rs, src/model.rs:3573-3860, :5180-5420) -------------

// Model facts of a GGUF file as the reference's loaders see them.
static int gguf_summary_impl(const char *path, RustyGgufSummary *out) {
    if (!path || !out) return 0;
    GgufFile G;
    if (!G.open_path(path)) {
        if (debug_on()) fprintf(stderr, "[rusty_hip] %s: %s\n", path, G.error.c_str());
        return 0;
    }
    GgufConfig c = gguf_config(G);
    memset(out, 0, sizeof(*out));
    snprintf(out->arch, sizeof(out->arch), "%s", c.arch.c_str());
    out->version = G.version;
    out->n_tensors = (uint32_t)G.tensors.size();
    out->data_offset = G.data_offset;
    out->n_layers = c.n_layers;
    out->dim = c.dim;
    out->n_heads = c.n_heads;
    out->n_kv_heads = c.n_kv;
    out->head_dim = c.head_dim;
    out->value_dim = c.value_dim;
    out->hidden_dim = c.hidden;
    out->vocab = c.vocab;
    out->context_length = c.ctx;
    out->sliding_window = c.window;
    out->n_experts = c.n_experts;
    out->top_k = c.top_k;
    out->rope_orig_ctx = c.rope_orig_ctx;
    out->rope_theta = c.theta;
    out->rms_eps = c.eps;
    out->rope_scaling = c.rope_scaling;
    // load_model's shape override of head_dim / value_dim (src/model.rs:3668-3724)
    for (uint32_t l = 0; l < c.n_layers && c.arch != "gpt-oss"; l++) {
        const GgufTensor *q = G.find("blk." + std::to_string(l) + ".attn_q.weight");
        const GgufTensor *v = G.find("blk." + std::to_string(l) + ".attn_v.weight");
        bool hq = false, hv = false;
        if (q && q->dims.size() >= 2 && q->dims[0] == c.dim && c.n_heads && q->dims[1] % c.n_heads == 0) {
            out->head_dim = (uint32_t)(q->dims[1] / c.n_heads);
            hq = true;
        }
        if (v && v->dims.size() >= 2 && v->dims[0] == c.dim && c.n_kv && v->dims[1] % c.n_kv == 0) {
            out->value_dim = (uint32_t)(v->dims[1] / c.n_kv);
            hv = true;
        }
        if (hq && hv) break;
    }
    out->tied_output = G.find("output.weight") ? 0 : 1;
    out->fused_qkv = G.find("blk.0.attn_qkv.weight") ? 1 : 0;
    out->qkv_bias = (G.find("blk.0.attn_q.bias") || G.find("blk.0.attn_qkv.bias")) ? 1 : 0;
    return 1;
}

// GGUF summary: a parse or allocation failure (std::bad_alloc included) returns 0
// instead of leaving through the C ABI.
int rusty_hip_gguf_summary(const char *path, RustyGgufSummary *out) {
    try {
        return gguf_summary_impl(path, out);
    } catch (...) {
        if (debug_on()) fprintf(stderr, "[rusty_hip] gguf_summary_impl: exception\n");
        return 0;
    }
}

}  // extern "C"

namespace rh {
// A float vector tensor (F32, F16 or BF16) as f32, n elements.
static bool gguf_f32(const GgufFile &G, const std::string &name, size_t n, std::vector<float> *out) {
    const GgufTensor *t = G.find(name);
    if (!t || t->numel() < n) return false;
    int64_t len;
    const uint8_t *p = G.data(*t, &len);
    if (!p) return false;
    out->resize(n);
    if (t->type == 0) {
        memcpy(out->data(), p, n * 4);
    } else if (t->type == 1) {
        for (size_t i = 0; i < n; i++) (*out)[i] = f16_to_f32_host((uint16_t)(p[2 * i] | (p[2 * i + 1] << 8)));
    } else if (t->type == 30) {
        for (size_t i = 0; i < n; i++) {
            uint32_t b = (uint32_t)(p[2 * i] | (p[2 * i + 1] << 8)) << 16;
            memcpy(&(*out)[i], &b, 4);
        }
    } else {
        return false;
    }
    return true;
}

struct GgufMat {
    const uint8_t *p = nullptr;
    int64_t len = 0, rows = 0, cols = 0;
    uint32_t type = 0;
};
// A 2-D (or expert-major 3-D) block tensor: rows = product of dims[1..].
static bool gguf_mat(const GgufFile &G, const std::string &name, GgufMat *m) {
    const GgufTensor *t = G.find(name);
    if (!t || t->dims.size() < 2) return false;
    m->p = G.data(*t, &m->len);
    if (!m->p) return false;
    m->cols = (int64_t)t->dims[0];
    m->rows = 1;
    for (size_t i = 1; i < t->dims.size(); i++) m->rows *= (int64_t)t->dims[i];
    m->type = t->type;
    return true;
}

static void gguf_note(const char *path, const std::string &what) {
    if (debug_on()) fprintf(stderr, "[rusty_hip] %s: %s\n", path, what.c_str());
}

// build_rope_inv_freq (src/model.rs:3031-3057) and build_rope_inv_freq_gpt_oss
// (:3059-3098) with libm powf / logf on f32, as Rust's f32::powf / ln.
static std::vector<float> rope_table(const GgufConfig &c, bool yarn, float *concentration) {
    const uint32_t half = c.head_dim / 2;
    std::vector<float> inv(half);
    *concentration = 1.0f;
    const bool scaled = yarn && c.rope_scaling > 1.0f;
    float lo = 0.0f, hi = 0.0f;
    if (scaled) {
        const float two_pi = 2.0f * 3.14159265358979323846f;
        const float dh = (float)c.head_dim / 2.0f;
        lo = dh * (logf((float)c.rope_orig_ctx / (32.0f * two_pi)) / logf(c.theta));
        hi = dh * (logf((float)c.rope_orig_ctx / two_pi) / logf(c.theta));
        *concentration = 0.1f * logf(c.rope_scaling) + 1.0f;
    }
    for (uint32_t i = 0; i < half; i++) {
        const float base = powf(c.theta, (float)(2 * i) / (float)c.head_dim);
        if (!yarn) {
            inv[i] = 1.0f / (1.0f * base * 1.0f);
        } else if (!scaled) {
            inv[i] = 1.0f / base;
        } else {
            float r = ((float)i - lo) / (hi - lo);
            r = std::min(1.0f, std::max(0.0f, r));
            const float keep = 1.0f - r;
            inv[i] = (1.0f / (c.rope_scaling * base)) * (1.0f - keep) + (1.0f / base) * keep;
        }
    }
    return inv;
}
}  // namespace rh

extern "C" {

static int resident_load_gguf_impl(const char *path, uint32_t max_len) {
    if (!path || max_len == 0) return 0;
    GgufFile G;
    if (!G.open_path(path)) {
        gguf_note(path, G.error);
        return 0;
    }
    GgufConfig c = gguf_config(G);
    auto blk = [](uint32_t l, const char *nm) { return "blk." + std::to_string(l) + "." + nm; };
    std::vector<std::vector<float>> keep;  // host vectors alive until each call has uploaded them
    auto vec = [&](const std::string &name, size_t n, const float **dst) {
        keep.emplace_back();
        if (!gguf_f32(G, name, n, &keep.back())) {
            gguf_note(path, "missing or bad f32 tensor " + name);
            return false;
        }
        *dst = keep.back().data();
        return true;
    };
    auto mat = [&](const std::string &name, GgufMat *m) {
        if (gguf_mat(G, name, m)) return true;
        gguf_note(path, "missing or bad tensor " + name);
        return false;
    };
    GgufMat emb, outw;
    if (!mat("token_embd.weight", &emb)) return 0;
    std::vector<float> out_norm;  // kept apart: `keep` is cleared after every layer
    if (!gguf_f32(G, "output_norm.weight", c.dim, &out_norm)) {
        gguf_note(path, "missing or bad f32 tensor output_norm.weight");
        return 0;
    }
    float conc = 1.0f;
    if (c.arch == "gpt-oss") {
        if (!mat("output.weight", &outw)) return 0;
        (void)rope_table(c, true, &conc);
        if (!rusty_hip_resident_configure_moe(c.n_layers, c.dim, c.n_heads, c.n_kv, c.head_dim, c.hidden,
                                              c.n_experts, c.top_k, c.vocab, max_len, c.window, c.eps, conc))
            return 0;
        for (uint32_t l = 0; l < c.n_layers; l++) {
            RustyMoeLayerDesc d;
            memset(&d, 0, sizeof(d));
            const char *wn[4] = {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight"};
            for (int i = 0; i < 4; i++) {
                GgufMat m;
                if (!mat(blk(l, wn[i]), &m)) return 0;
                d.w[i] = m.p;
                d.w_len[i] = (uintptr_t)m.len;
                d.w_dt[i] = m.type;
            }
            const uint32_t qd = c.n_heads * c.head_dim, kd = c.n_kv * c.head_dim;
            if (!vec(blk(l, "attn_q.bias"), qd, &d.bq) || !vec(blk(l, "attn_k.bias"), kd, &d.bk) ||
                !vec(blk(l, "attn_v.bias"), kd, &d.bv) || !vec(blk(l, "attn_output.bias"), c.dim, &d.bo) ||
                !vec(blk(l, "attn_sinks.weight"), c.n_heads, &d.sinks) ||
                !vec(blk(l, "attn_norm.weight"), c.dim, &d.attn_norm) ||
                !vec(blk(l, "post_attention_norm.weight"), c.dim, &d.post_attn_norm) ||
                !vec(blk(l, "ffn_gate_inp.bias"), c.n_experts, &d.router_bias))
                return 0;
            GgufMat r;
            if (!mat(blk(l, "ffn_gate_inp.weight"), &r)) return 0;
            d.router = r.p;
            d.router_len = (uintptr_t)r.len;
            d.router_dt = r.type;
            const char *en[3] = {"ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight"};
            const char *bn[3] = {"ffn_gate_exps.bias", "ffn_up_exps.bias", "ffn_down_exps.bias"};
            const size_t bl[3] = {(size_t)c.n_experts * c.hidden, (size_t)c.n_experts * c.hidden,
                                  (size_t)c.n_experts * c.dim};
            for (int i = 0; i < 3; i++) {
                GgufMat m;
                if (!mat(blk(l, en[i]), &m)) return 0;
                d.exps[i] = m.p;
                d.exps_len[i] = (uintptr_t)m.len;
                d.exps_dt = m.type;
                if (!vec(blk(l, bn[i]), bl[i], &d.exps_bias[i])) return 0;
            }
            if (!rusty_hip_resident_set_moe_layer(l, &d)) return 0;
            keep.clear();
        }
    } else {
        // load_model (src/model.rs:3573-3860): head / value dims from the
        // attn_q / attn_v shapes, fused attn_qkv split by rows, tied output
        for (uint32_t l = 0; l < c.n_layers; l++) {
            const GgufTensor *q = G.find(blk(l, "attn_q.weight")), *v = G.find(blk(l, "attn_v.weight"));
            bool hq = false, hv = false;
            if (q && q->dims.size() >= 2 && q->dims[0] == c.dim && c.n_heads && q->dims[1] % c.n_heads == 0) {
                c.head_dim = (uint32_t)(q->dims[1] / c.n_heads);
                hq = true;
            }
            if (v && v->dims.size() >= 2 && v->dims[0] == c.dim && c.n_kv && v->dims[1] % c.n_kv == 0) {
                c.value_dim = (uint32_t)(v->dims[1] / c.n_kv);
                hv = true;
            }
            if (hq && hv) break;
        }
        const bool neox = c.arch == "qwen2" || c.arch == "qwen3";
        if (!rusty_hip_resident_configure(c.n_layers, c.dim, c.n_heads, c.n_kv, c.head_dim, c.value_dim, c.hidden,
                                          c.vocab, max_len, c.eps, neox ? 1 : 0))
            return 0;
        const uint32_t rows[7] = {c.n_heads * c.head_dim, c.n_kv * c.head_dim, c.n_kv * c.value_dim, c.dim,
                                  c.hidden, c.hidden, c.dim};
        for (uint32_t l = 0; l < c.n_layers; l++) {
            RustyResidentLayerDesc d;
            memset(&d, 0, sizeof(d));
            if (G.find(blk(l, "attn_q.weight"))) {
                const char *nm[3] = {"attn_q.weight", "attn_k.weight", "attn_v.weight"};
                const char *bn[3] = {"attn_q.bias", "attn_k.bias", "attn_v.bias"};
                const float **bd[3] = {&d.bq, &d.bk, &d.bv};
                uint32_t *bln[3] = {&d.bq_len, &d.bk_len, &d.bv_len};
                for (int i = 0; i < 3; i++) {
                    GgufMat m;
                    if (!mat(blk(l, nm[i]), &m)) return 0;
                    d.w[i] = m.p;
                    d.w_len[i] = (uintptr_t)m.len;
                    d.w_rows[i] = (uint32_t)m.rows;
                    d.w_dt[i] = m.type;
                    if (G.find(blk(l, bn[i]))) {
                        if (!vec(blk(l, bn[i]), rows[i], bd[i])) return 0;
                        *bln[i] = rows[i];
                    }
                }
            } else {
                GgufMat m;
                if (!mat(blk(l, "attn_qkv.weight"), &m)) return 0;
                const int64_t rb = row_bytes_of((int)m.type, m.cols);
                if (rb <= 0 || m.rows != (int64_t)rows[0] + rows[1] + rows[2]) {
                    gguf_note(path, "attn_qkv rows do not split into q/k/v");
                    return 0;
                }
                const float *qkv_b = nullptr;
                const bool has_b = G.find(blk(l, "attn_qkv.bias")) != nullptr;
                if (has_b && !vec(blk(l, "attn_qkv.bias"), (size_t)m.rows, &qkv_b)) return 0;
                int64_t r0 = 0;
                const float **bd[3] = {&d.bq, &d.bk, &d.bv};
                uint32_t *bln[3] = {&d.bq_len, &d.bk_len, &d.bv_len};
                for (int i = 0; i < 3; i++) {
                    d.w[i] = m.p + r0 * rb;
                    d.w_len[i] = (uintptr_t)(rows[i] * rb);
                    d.w_rows[i] = rows[i];
                    d.w_dt[i] = m.type;
                    if (has_b) {
                        *bd[i] = qkv_b + r0;
                        *bln[i] = rows[i];
                    }
                    r0 += rows[i];
                }
            }
            const char *on[4] = {"attn_output.weight", "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"};
            for (int i = 0; i < 4; i++) {
                GgufMat m;
                if (!mat(blk(l, on[i]), &m)) return 0;
                d.w[3 + i] = m.p;
                d.w_len[3 + i] = (uintptr_t)m.len;
                d.w_rows[3 + i] = (uint32_t)m.rows;
                d.w_dt[3 + i] = m.type;
            }
            if (!vec(blk(l, "attn_norm.weight"), c.dim, &d.attn_norm) ||
                !vec(blk(l, "ffn_norm.weight"), c.dim, &d.ffn_norm))
                return 0;
            if (!rusty_hip_resident_set_layer(l, &d)) return 0;
            keep.clear();
        }
        if (G.find("output.weight")) {
            if (!mat("output.weight", &outw)) return 0;
        } else {
            outw = emb;  // output tied to the embedding (src/model.rs:3653-3667)
        }
    }
    std::vector<float> inv = rope_table(c, c.arch == "gpt-oss", &conc);
    if (!rusty_hip_resident_set_output(out_norm.data(), outw.p, (uintptr_t)outw.len, (uint32_t)outw.rows, outw.type,
                                       inv.data(), (uint32_t)inv.size()))
        return 0;
    if (!rusty_hip_resident_set_embedding(emb.p, (uintptr_t)emb.len, emb.type)) return 0;
    return 1;
}

// GGUF resident load: a parse or allocation failure (std::bad_alloc included) returns 0
// instead of leaving through the C ABI.
int rusty_hip_resident_load_gguf(const char *path, uint32_t max_len) {
    try {
        return resident_load_gguf_impl(path, max_len);
    } catch (...) {
        if (debug_on()) fprintf(stderr, "[rusty_hip] resident_load_gguf_impl: exception\n");
        return 0;
    }
}

}  // extern "C"
