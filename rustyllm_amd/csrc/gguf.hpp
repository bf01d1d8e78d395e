// gguf.hpp — native GGUF v3 reader and the resident decoder's file loader.
//
// The parse follows GGUFFile::parse (src/gguf.rs:338-418): magic "GGUF", u32
// version, u64 tensor and metadata counts, typed metadata values (0-12,
// arrays nested), tensor infos (name, dims fastest first, GGML type, offset
// from the data start), data from the first multiple of general.alignment
// (default 32) after the header.  Config::from_gguf (src/model.rs:40-120)
// reads the model shape from it; the loader then names tensors as load_model
// (:3573-3860: tied output, head/value dim from the attn_q / attn_v shapes,
// fused attn_qkv split by rows) or load_gpt_oss_model (:5180-5420) do, and
// hands them to the resident decoder through the same exports a host would
// call.  The file is mapped read-only; weights go from the mapping through
// two pinned staging buffers to their row-padded device copies, so page-in of
// the next chunk overlaps the DMA of the last.
#pragma once
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

namespace rh {

enum : uint32_t {
    GV_U8 = 0, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64
};

struct GgufValue {
    uint32_t type = 0;
    uint64_t u = 0;  // integers and bools, as stored (sign-extended for signed types)
    double f = 0.0;  // f32 / f64
    std::string s;
    std::vector<GgufValue> arr;

    // MetaValue::as_u32 (src/gguf.rs:131-141): integer types wrap to u32
    bool as_u32(uint32_t *out) const {
        switch (type) {
        case GV_U8: case GV_U16: case GV_U32: case GV_I32: case GV_U64: case GV_I64:
            *out = (uint32_t)u;
            return true;
        default: return false;
        }
    }
    // one element of MetaValue::as_u32_array (src/gguf.rs:188-207): negative
    // entries and 64-bit values above u32::MAX are dropped, not wrapped
    bool as_u32_elem(uint32_t *out) const {
        switch (type) {
        case GV_U8: case GV_U16: case GV_U32:
            *out = (uint32_t)u;
            return true;
        case GV_I8: case GV_I16: case GV_I32: case GV_I64:
            if ((int64_t)u < 0 || (int64_t)u > (int64_t)0xFFFFFFFFll) return false;
            *out = (uint32_t)u;
            return true;
        case GV_U64:
            if (u > 0xFFFFFFFFull) return false;
            *out = (uint32_t)u;
            return true;
        default: return false;
        }
    }
    bool as_f32(float *out) const {
        if (type != GV_F32 && type != GV_F64) return false;
        *out = (float)f;
        return true;
    }
};

struct GgufTensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
    uint64_t numel() const {
        uint64_t n = 1;
        for (uint64_t d : dims) n *= d;
        return n;
    }
};

// IEEE binary16 -> binary32 (exact; subnormals, infinities and NaN kept).
static inline float f16_to_f32_host(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {  // subnormal: normalise
        int e = -1;
        do {
            man <<= 1;
            e++;
        } while ((man & 0x400u) == 0);
        bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// (elements, bytes) per block of a GGML type (GGMLType::block_size /
// block_bytes, src/gguf.rs:59-87); {0, 0} when unsupported.
static inline void ggml_block(uint32_t t, int64_t *elems, int64_t *bytes) {
    switch (t) {
    case 0: *elems = 1; *bytes = 4; return;
    case 1: case 30: *elems = 1; *bytes = 2; return;
    case 2: *elems = 32; *bytes = 18; return;
    case 3: *elems = 32; *bytes = 20; return;
    case 6: *elems = 32; *bytes = 22; return;
    case 7: *elems = 32; *bytes = 24; return;
    case 8: *elems = 32; *bytes = 34; return;
    case 9: *elems = 32; *bytes = 36; return;
    case 12: *elems = 256; *bytes = 144; return;
    case 13: *elems = 256; *bytes = 176; return;
    case 14: *elems = 256; *bytes = 210; return;
    case 39: *elems = 32; *bytes = 17; return;
    default: *elems = 0; *bytes = 0; return;
    }
}
// GGMLType::data_size (src/gguf.rs:89-107), -1 when unsupported
static inline int64_t ggml_data_size(uint32_t t, uint64_t n) {
    int64_t be, bb;
    ggml_block(t, &be, &bb);
    if (be == 0) return -1;
    return (int64_t)((n + (uint64_t)be - 1) / (uint64_t)be) * bb;
}

class GgufFile {
  public:
    std::unordered_map<std::string, GgufValue> meta;
    std::vector<GgufTensor> tensors;
    std::unordered_map<std::string, size_t> index;
    uint32_t version = 0;
    size_t data_offset = 0;
    const uint8_t *base = nullptr;
    size_t size = 0;
    std::string error;

    ~GgufFile() {
        if (base) munmap((void *)base, size);
        if (fd >= 0) close(fd);
    }

    bool open_path(const char *path) {
        fd = ::open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) return fail("cannot open file");
        struct stat st;
        if (fstat(fd, &st) != 0) return fail("cannot stat file");
        size = (size_t)st.st_size;
        if (size < 4) return fail("File too small for GGUF header");
        void *m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) return fail("mmap failed");
        base = (const uint8_t *)m;
        (void)madvise(m, size, MADV_SEQUENTIAL);
        return parse();
    }

    const GgufTensor *find(const std::string &name) const {
        auto it = index.find(name);
        return it == index.end() ? nullptr : &tensors[it->second];
    }
    // The tensor's bytes (data_size of its elements) inside the mapping, or
    // null when the type is unsupported or the range leaves the file.
    const uint8_t *data(const GgufTensor &t, int64_t *len) const {
        int64_t n = ggml_data_size(t.type, t.numel());
        if (n < 0) return nullptr;
        uint64_t start = (uint64_t)data_offset + t.offset;
        if (start > size || (uint64_t)n > size - start) return nullptr;
        *len = n;
        return base + start;
    }
    uint32_t get_u32(const std::string &k, uint32_t def) const {
        auto it = meta.find(k);
        uint32_t v;
        return (it != meta.end() && it->second.as_u32(&v)) ? v : def;
    }
    float get_f32(const std::string &k, float def) const {
        auto it = meta.find(k);
        float v;
        return (it != meta.end() && it->second.as_f32(&v)) ? v : def;
    }
    std::string get_str(const std::string &k) const {
        auto it = meta.find(k);
        return (it != meta.end() && it->second.type == GV_STR) ? it->second.s : std::string();
    }
    const GgufValue *get(const std::string &k) const {
        auto it = meta.find(k);
        return it == meta.end() ? nullptr : &it->second;
    }

  private:
    int fd = -1;
    size_t pos = 0;

    bool fail(const char *m) {
        if (error.empty()) error = m;
        return false;
    }
    bool need(size_t n) {
        if (pos > size || n > size - pos) return fail("truncated GGUF header");
        return true;
    }
    size_t remaining() const { return pos > size ? 0 : size - pos; }
    // Fewest bytes one encoded value of a metadata type can take; 0 for an
    // unknown type.  A count is accepted only if that many values could fit
    // in the bytes left, so a corrupt count cannot make the parser reserve
    // memory the file could never fill.
    static size_t min_value_bytes(uint32_t t) {
        switch (t) {
        case GV_U8: case GV_I8: case GV_BOOL: return 1;
        case GV_U16: case GV_I16: return 2;
        case GV_U32: case GV_I32: case GV_F32: return 4;
        case GV_U64: case GV_I64: case GV_F64: return 8;
        case GV_STR: return 8;   // the length prefix
        case GV_ARR: return 12;  // element type + count
        default: return 0;
        }
    }
    template <class T>
    bool rd(T *v) {
        if (!need(sizeof(T))) return false;
        memcpy(v, base + pos, sizeof(T));  // little-endian host
        pos += sizeof(T);
        return true;
    }
    bool rd_str(std::string *s) {
        uint64_t n;
        if (!rd(&n) || !need((size_t)n)) return false;
        s->assign((const char *)base + pos, (size_t)n);
        pos += (size_t)n;
        return true;
    }
    bool rd_value(uint32_t t, GgufValue *v, int depth) {
        v->type = t;
        switch (t) {
        case GV_U8: case GV_BOOL: { uint8_t x; if (!rd(&x)) return false; v->u = x; return true; }
        case GV_I8: { int8_t x; if (!rd(&x)) return false; v->u = (uint64_t)(int64_t)x; return true; }
        case GV_U16: { uint16_t x; if (!rd(&x)) return false; v->u = x; return true; }
        case GV_I16: { int16_t x; if (!rd(&x)) return false; v->u = (uint64_t)(int64_t)x; return true; }
        case GV_U32: { uint32_t x; if (!rd(&x)) return false; v->u = x; return true; }
        case GV_I32: { int32_t x; if (!rd(&x)) return false; v->u = (uint64_t)(int64_t)x; return true; }
        case GV_U64: { uint64_t x; if (!rd(&x)) return false; v->u = x; return true; }
        case GV_I64: { int64_t x; if (!rd(&x)) return false; v->u = (uint64_t)x; return true; }
        case GV_F32: { float x; if (!rd(&x)) return false; v->f = x; return true; }
        case GV_F64: { double x; if (!rd(&x)) return false; v->f = x; return true; }
        case GV_STR: return rd_str(&v->s);
        case GV_ARR: {
            uint32_t et;
            uint64_t n;
            if (depth > 8 || !rd(&et) || !rd(&n)) return fail("bad GGUF array");
            const size_t mb = min_value_bytes(et);
            if (mb == 0) return fail("Unknown GGUF metadata value type");
            if (n > remaining() / mb) return fail("bad GGUF array length");
            v->arr.resize((size_t)n);
            for (uint64_t i = 0; i < n; i++)
                if (!rd_value(et, &v->arr[(size_t)i], depth + 1)) return false;
            return true;
        }
        default: return fail("Unknown GGUF metadata value type");
        }
    }
    bool parse() {
        if (memcmp(base, "GGUF", 4) != 0) return fail("Invalid GGUF magic");
        pos = 4;
        uint64_t n_tensors, n_kv;
        if (!rd(&version) || !rd(&n_tensors) || !rd(&n_kv)) return false;
        // a key/value pair takes at least 8 + 4 + 1 bytes, a tensor info
        // 8 (name length) + 4 (rank) + 4 (type) + 8 (offset)
        if (n_kv > remaining() / 13) return fail("bad GGUF counts");
        for (uint64_t i = 0; i < n_kv; i++) {
            std::string key;
            uint32_t t;
            GgufValue v;
            if (!rd_str(&key) || !rd(&t) || !rd_value(t, &v, 0)) return false;
            meta[key] = std::move(v);
        }
        if (n_tensors > remaining() / 24) return fail("bad GGUF counts");
        tensors.resize((size_t)n_tensors);
        for (uint64_t i = 0; i < n_tensors; i++) {
            GgufTensor &T = tensors[(size_t)i];
            uint32_t nd;
            if (!rd_str(&T.name) || !rd(&nd)) return false;
            if (nd > 8) return fail("bad tensor rank");
            T.dims.resize(nd);
            for (uint32_t d = 0; d < nd; d++)
                if (!rd(&T.dims[d])) return false;
            if (!rd(&T.type) || !rd(&T.offset)) return false;
            index[T.name] = (size_t)i;
        }
        uint32_t align = get_u32("general.alignment", 32);
        if (align == 0) return fail("bad alignment");
        data_offset = (pos + align - 1) / align * align;
        return true;
    }
};

// Config::from_gguf (src/model.rs:40-120) for the fields the decoders use.
struct GgufConfig {
    std::string arch;
    uint32_t dim = 0, hidden = 0, n_layers = 0, n_heads = 0, n_kv = 0, vocab = 0, ctx = 2048;
    uint32_t head_dim = 0, value_dim = 0, window = 0, n_experts = 0, top_k = 0, rope_orig_ctx = 0;
    float theta = 10000.0f, eps = 1e-5f, rope_scaling = 1.0f;
};

static GgufConfig gguf_config(const GgufFile &G) {
    GgufConfig c;
    c.arch = G.get_str("general.architecture");
    if (c.arch.empty()) c.arch = "llama";
    const std::string p = c.arch + ".";
    c.dim = G.get_u32(p + "embedding_length", 0);
    c.n_heads = G.get_u32(p + "attention.head_count", 0);
    if (const GgufValue *hc = G.get(p + "attention.head_count"))
        if (hc->type == GV_ARR)
            for (const GgufValue &e : hc->arr) {
                uint32_t v;
                if (e.as_u32_elem(&v)) c.n_heads = std::max(c.n_heads, v);
            }
    c.n_kv = G.get_u32(p + "attention.head_count_kv", c.n_heads);
    const uint32_t rope_dim = G.get_u32(p + "rope.dimension_count", 0);
    const uint32_t def_hd = (c.dim > 0 && c.n_heads > 0) ? c.dim / c.n_heads : rope_dim;
    c.head_dim = G.get_u32(p + "attention.key_length", def_hd);
    c.value_dim = G.get_u32(p + "attention.value_length", c.head_dim);
    c.vocab = G.get_u32(p + "vocab_size", 0);
    if (const GgufValue *tk = G.get("tokenizer.ggml.tokens"))
        if (tk->type == GV_ARR) {  // as_string_array: string entries only
            uint32_t n = 0;
            for (const GgufValue &e : tk->arr) n += e.type == GV_STR ? 1u : 0u;
            c.vocab = std::max(c.vocab, n);
        }
    if (const GgufValue *ff = G.get(p + "feed_forward_length")) {
        uint32_t v;
        if (ff->as_u32(&v)) {
            c.hidden = v;
        } else if (ff->type == GV_ARR) {
            for (const GgufValue &e : ff->arr)
                if (e.as_u32(&v)) c.hidden = std::max(c.hidden, v);
        }
    }
    c.n_layers = G.get_u32(p + "block_count", 0);
    c.ctx = G.get_u32(p + "context_length", 2048);
    c.theta = G.get_f32(p + "rope.freq_base", 10000.0f);
    c.eps = G.get_f32(p + "attention.layer_norm_rms_epsilon", 1e-5f);
    c.window = G.get_u32(p + "attention.sliding_window", 0);
    c.n_experts = G.get_u32(p + "expert_count", 0);
    c.top_k = G.get_u32(p + "expert_used_count", 0);
    c.rope_scaling = G.get_f32(p + "rope.scaling.factor", 1.0f);
    c.rope_orig_ctx = G.get_u32(p + "rope.scaling.original_context_length", 0);
    return c;
}

}  // namespace rh
