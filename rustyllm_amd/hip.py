"""ctypes binding of librusty_hip.so (include/rusty_hip.h).

The functions mirror the safe wrappers of the reference's backend seam
(src/metal.rs): each returns True when the device wrote the full output and
False when the caller must run its CPU kernel (src/metal.rs:716-720).
`RUSTY_HIP=0` in the environment disables dispatch, as RUSTY_LLM_METAL=0 does
for the reference (src/metal.rs:586-631).

Importing this module loads the library and raises if it is missing: there is
no silent fallback inside the product path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import build as _build

LIB_PATH = _build.HIP_LIB
SYMBOLS = [
    "rusty_hip_available", "rusty_hip_q4k_matvec", "rusty_hip_q6k_matvec", "rusty_hip_q6k_matvec2",
    "rusty_hip_q6k_matvec3", "rusty_hip_q4k_matvec2", "rusty_hip_q4k_matvec3", "rusty_hip_q4k_q4k_q6k_matvec3",
    "rusty_hip_q4k_q4k_q6k_ffn", "rusty_hip_mistral_post_attention_ffn", "rusty_hip_q8_0_matvec",
    "rusty_hip_attention", "rusty_hip_resident_configure", "rusty_hip_resident_set_layer",
    "rusty_hip_resident_set_output", "rusty_hip_resident_decode", "rusty_hip_mxfp4_matvec",
    "rusty_hip_mxfp4_matvec2", "rusty_hip_matvec", "rusty_hip_resident_set_embedding",
    "rusty_hip_resident_generate", "rusty_hip_resident_kv_read", "rusty_hip_resident_kv_write", "rusty_hip_sync",
    "rusty_hip_profile_enable", "rusty_hip_profile_get", "rusty_hip_resident_time_decode",
    "rusty_hip_debug_quantize_q8k", "rusty_hip_debug_dequant", "rusty_hip_debug_block_ints",
    "rusty_hip_debug_rmsnorm", "rusty_hip_debug_silu_mul", "rusty_hip_debug_rope", "rusty_hip_debug_greedy",
    "rusty_hip_debug_f16", "rusty_hip_weight_cache_clear", "rusty_hip_attention_mode", "rusty_hip_debug_expf",
    "rusty_hip_moe_ffn", "rusty_hip_resident_configure_moe", "rusty_hip_resident_set_moe_layer",
    "rusty_hip_kquant_matvec_batch", "rusty_hip_resident_prefill", "rusty_hip_bench_matvec",
    "rusty_hip_bench_attention", "rusty_hip_attention_noalloc", "rusty_hip_gguf_summary",
    "rusty_hip_resident_load_gguf", "rusty_hip_resident_enable_bf16", "rusty_hip_debug_stream_mark",
    "rusty_hip_set_expert_mfma", "rusty_hip_mxfp4_experts",
]


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc, gfx950)")
    return C.CDLL(LIB_PATH)


lib = _load()
_p, _u, _f, _i = C.c_void_p, C.c_size_t, C.c_float, C.c_int
_u32, _i64 = C.c_uint32, C.c_int64


def _sig(name, res, *args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = list(args)


_sig("rusty_hip_available", _i)
for _n in ("rusty_hip_q4k_matvec", "rusty_hip_q6k_matvec", "rusty_hip_q8_0_matvec", "rusty_hip_mxfp4_matvec"):
    _sig(_n, _i, _p, _u, _p, _u, _u, _p)
_sig("rusty_hip_matvec", _i, _u32, _p, _u, _p, _u, _u, _p)
for _n in ("rusty_hip_q6k_matvec2", "rusty_hip_q4k_matvec2", "rusty_hip_mxfp4_matvec2"):
    _sig(_n, _i, _p, _u, _u, _p, _u, _u, _p, _u, _p, _p)
for _n in ("rusty_hip_q6k_matvec3", "rusty_hip_q4k_matvec3", "rusty_hip_q4k_q4k_q6k_matvec3"):
    _sig(_n, _i, _p, _u, _u, _p, _u, _u, _p, _u, _u, _p, _u, _p, _p, _p)
_sig("rusty_hip_q4k_q4k_q6k_ffn", _i, _p, _u, _p, _u, _p, _u, _p, _u, _u, _u, _u, _p)
_sig("rusty_hip_mistral_post_attention_ffn", _i, _p, _u, _p, _u, _p, _u, _p, _u, _p, _u, _p, _u, _p, _f, _u, _u, _u)
_sig("rusty_hip_attention", _i, _p, _u, _p, _u, _p, _u, _p, _u, _p, _u, _u, _u, _u, _u, _u, _u, _u, _u, _u, _f, _i)
_sig("rusty_hip_attention_noalloc", _i, _p, _u, _p, _u, _p, _u, _p, _u, _p, _u, _u, _u, _u, _u, _u, _u, _u, _u, _u, _f,
     _i)
_sig("rusty_hip_resident_configure", _i, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _f, _u32)
_sig("rusty_hip_resident_set_layer", _i, _u32, _p)
_sig("rusty_hip_resident_set_output", _i, _p, _p, _u, _u32, _u32, _p, _u32)
_sig("rusty_hip_resident_decode", _i, _p, _u32, _u32, _i, _p)
_sig("rusty_hip_resident_set_embedding", _i, _p, _u, _u32)
_sig("rusty_hip_resident_generate", _i, _p, _u32, _u32, _u32, _f, _p, _p)
_sig("rusty_hip_resident_kv_read", _i, _u32, _u32, _u32, _u32, _p)
_sig("rusty_hip_resident_kv_write", _i, _u32, _u32, _u32, _u32, _p)
_sig("rusty_hip_sync", _i)
_sig("rusty_hip_weight_cache_clear", _i)
_sig("rusty_hip_attention_mode", _i, _i)
_sig("rusty_hip_debug_expf", _i, _p, _u, _p)
_sig("rusty_hip_profile_enable", _i, _i)
_sig("rusty_hip_profile_get", _i, _i, C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_int64))
_sig("rusty_hip_resident_time_decode", _i, _u32, _f, C.POINTER(C.c_double))
_sig("rusty_hip_debug_quantize_q8k", _i, _p, _u, _p, _p, _p)
_sig("rusty_hip_debug_dequant", _i, _u32, _p, _u, _u, _u, _p)
_sig("rusty_hip_debug_block_ints", _i, _u32, _p, _u, _u, _u, _p, _p)
_sig("rusty_hip_debug_rmsnorm", _i, _p, _p, _f, _u, _p)
_sig("rusty_hip_debug_silu_mul", _i, _p, _p, _u, _p)
_sig("rusty_hip_debug_rope", _i, _p, _p, _u32, _u32, _u32, _u32, _p, _u32)
_sig("rusty_hip_debug_greedy", _i, _p, _u, _p, _u32, _f, _p)
_sig("rusty_hip_debug_f16", _i, _p, _u, _p)
_sig("rusty_hip_debug_stream_mark", _i)
_sig("rusty_hip_set_expert_mfma", _i, _i)
_sig("rusty_hip_mxfp4_experts", _i, _p, _i64, _i64, _u32, _u32, _u32, _p, _i64, _i, _u32, _p, _u32, _p, _i64, _i)
_sig("rusty_hip_resident_configure_moe", _i, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _f,
     _f)
_sig("rusty_hip_resident_set_moe_layer", _i, _u32, _p)
_sig("rusty_hip_kquant_matvec_batch", _i, _u32, _p, _u, _u, _u, _p, _u, _p, _u)
_sig("rusty_hip_resident_prefill", _i, _p, _u32, _u32)
_sig("rusty_hip_bench_matvec", _i, _u32, _p, _u, _p, _u, _u, _u32, _u32, _p)
_sig("rusty_hip_bench_attention", _i, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _i, _p)
_sig("rusty_hip_moe_ffn", _i, _p, _u, _p, _u, _u32, _p, _u32, _u32, _p, _u, _p, _u, _p, _u, _u32, _u, _p, _p, _p, _p,
     _p, _p)



class GgufSummary(C.Structure):
    _fields_ = [("arch", C.c_char * 32), ("version", C.c_uint32), ("n_tensors", C.c_uint32),
                ("data_offset", C.c_uint64), ("n_layers", C.c_uint32), ("dim", C.c_uint32), ("n_heads", C.c_uint32),
                ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("value_dim", C.c_uint32),
                ("hidden_dim", C.c_uint32), ("vocab", C.c_uint32), ("context_length", C.c_uint32),
                ("sliding_window", C.c_uint32), ("n_experts", C.c_uint32), ("top_k", C.c_uint32),
                ("rope_orig_ctx", C.c_uint32), ("rope_theta", C.c_float), ("rms_eps", C.c_float),
                ("rope_scaling", C.c_float), ("tied_output", C.c_uint32), ("fused_qkv", C.c_uint32),
                ("qkv_bias", C.c_uint32)]


_sig("rusty_hip_gguf_summary", _i, C.c_char_p, C.POINTER(GgufSummary))
_sig("rusty_hip_resident_load_gguf", _i, C.c_char_p, _u32)
_sig("rusty_hip_resident_enable_bf16", _i, _i)


def gguf_summary(path: str):
    """The library's native parse of a GGUF file (host only), or None."""
    s = GgufSummary()
    if lib.rusty_hip_gguf_summary(os.fsencode(path), C.byref(s)) != 1:
        return None
    return s


Q8_0, Q4_K, Q6_K, MXFP4 = 8, 12, 14, 39


def enabled() -> bool:
    return os.environ.get("RUSTY_HIP", "1").strip().lower() not in ("0", "false", "off")


def available() -> bool:
    return enabled() and lib.rusty_hip_available() == 1


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    return a


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.uint8)


# ---- single / fused matvecs (src/metal.rs:709-935, 1523-1606) ---------------------
def matvec_into(ggml_type: int, weights: np.ndarray, x: np.ndarray, rows: int, cols: int, out: np.ndarray) -> bool:
    """Weight::matvec_into for one quantized weight (model.rs:218-257)."""
    if not enabled():
        return False
    w, xx = _u8(weights), _f32(x)
    assert out.dtype == np.float32 and out.flags.c_contiguous and out.size >= rows
    return lib.rusty_hip_matvec(ggml_type, _ptr(w), w.nbytes, _ptr(xx), rows, cols, _ptr(out)) == 1


def kquant_matvec_batch_into(kind: int, weights: np.ndarray, rows: int, cols: int, inputs: np.ndarray,
                             out: np.ndarray) -> bool:
    """matvec_kquant_batch_into (simd.rs:3417-3435): inputs [T][cols] row-major,
    out [T][rows] row-major; kind is Q4_K / Q6_K (GGML id or 0/1)."""
    if not enabled():
        return False
    w, xx = _u8(weights), _f32(inputs)
    assert out.dtype == np.float32 and out.flags.c_contiguous
    return lib.rusty_hip_kquant_matvec_batch(kind, _ptr(w), w.nbytes, rows, cols, _ptr(xx), xx.nbytes, _ptr(out),
                                             out.nbytes) == 1


def q4k_matvec_into(weights, x, rows, cols, out) -> bool:
    return matvec_into(Q4_K, weights, x, rows, cols, out)


def q6k_matvec_into(weights, x, rows, cols, out) -> bool:
    return matvec_into(Q6_K, weights, x, rows, cols, out)


def q8_0_matvec_into(weights, x, rows, cols, out) -> bool:
    return matvec_into(Q8_0, weights, x, rows, cols, out)


def mxfp4_matvec_into(weights, x, rows, cols, out) -> bool:
    return matvec_into(MXFP4, weights, x, rows, cols, out)


_FUSED3 = {(Q4_K, Q4_K, Q4_K): "rusty_hip_q4k_matvec3", (Q6_K, Q6_K, Q6_K): "rusty_hip_q6k_matvec3",
           (Q4_K, Q4_K, Q6_K): "rusty_hip_q4k_q4k_q6k_matvec3"}
_FUSED2 = {(Q4_K, Q4_K): "rusty_hip_q4k_matvec2", (Q6_K, Q6_K): "rusty_hip_q6k_matvec2",
           (MXFP4, MXFP4): "rusty_hip_mxfp4_matvec2"}


def quant_matvec3_into(a, b, c, x, cols, outs) -> bool:
    """try_quant_matvec3_into (model.rs:323-489): three projections, one activation.
    a/b/c are (weights, ggml_type, rows)."""
    if not enabled():
        return False
    name = _FUSED3.get((a[1], b[1], c[1]))
    if name is None:
        return False
    xx = _f32(x)
    ws = [_u8(m[0]) for m in (a, b, c)]
    fn = getattr(lib, name)
    return fn(_ptr(ws[0]), ws[0].nbytes, a[2], _ptr(ws[1]), ws[1].nbytes, b[2], _ptr(ws[2]), ws[2].nbytes, c[2],
              _ptr(xx), cols, _ptr(outs[0]), _ptr(outs[1]), _ptr(outs[2])) == 1


def quant_matvec2_into(a, b, x, cols, outs) -> bool:
    if not enabled():
        return False
    name = _FUSED2.get((a[1], b[1]))
    if name is None:
        return False
    xx = _f32(x)
    ws = [_u8(m[0]) for m in (a, b)]
    fn = getattr(lib, name)
    return fn(_ptr(ws[0]), ws[0].nbytes, a[2], _ptr(ws[1]), ws[1].nbytes, b[2], _ptr(xx), cols, _ptr(outs[0]),
              _ptr(outs[1])) == 1


def q4k_q4k_q6k_ffn_into(gate, up, down, x, input_cols, hidden_rows, down_rows, down_cols, out) -> bool:
    if not enabled():
        return False
    g_, u_, d_, xx = _u8(gate), _u8(up), _u8(down), _f32(x)
    return lib.rusty_hip_q4k_q4k_q6k_ffn(_ptr(g_), g_.nbytes, _ptr(u_), u_.nbytes, _ptr(d_), d_.nbytes, _ptr(xx),
                                         input_cols, hidden_rows, down_rows, down_cols, _ptr(out)) == 1


def mistral_post_attention_ffn_into(wo, gate, up, down, x, dim, attn_out, attn_cols, ffn_norm, eps, hidden_rows,
                                    down_rows, down_cols) -> bool:
    if not enabled():
        return False
    o_, g_, u_, d_ = _u8(wo), _u8(gate), _u8(up), _u8(down)
    a_, n_ = _f32(attn_out), _f32(ffn_norm)
    assert x.dtype == np.float32 and x.flags.c_contiguous
    return lib.rusty_hip_mistral_post_attention_ffn(_ptr(o_), o_.nbytes, _ptr(g_), g_.nbytes, _ptr(u_), u_.nbytes,
                                                    _ptr(d_), d_.nbytes, _ptr(x), dim, _ptr(a_), attn_cols, _ptr(n_),
                                                    eps, hidden_rows, down_rows, down_cols) == 1


# ---- attention (src/metal.rs:635-706) ------------------------------------------------
def _attention(query, keys, values, sinks, out, heads, kv_mul, head_dim, value_dim, key_stride, value_stride,
               slot_count, start_t, end_t, scale) -> bool:
    if not enabled():
        return False
    q, k, v = _f32(query), _f32(keys), _f32(values)
    s = _f32(sinks) if sinks is not None else None
    assert out.dtype == np.float32 and out.flags.c_contiguous
    return lib.rusty_hip_attention(_ptr(q), q.nbytes, _ptr(k), k.nbytes, _ptr(v), v.nbytes,
                                   _ptr(s) if s is not None else None, s.nbytes if s is not None else 0, _ptr(out),
                                   out.nbytes, heads, kv_mul, head_dim, value_dim, key_stride, value_stride,
                                   slot_count, start_t, end_t, scale, 1 if s is not None else 0) == 1


def attention_into(query, keys, values, out, heads, kv_mul, head_dim, value_dim, key_stride, value_stride,
                   slot_count, start_t, end_t, scale) -> bool:
    return _attention(query, keys, values, None, out, heads, kv_mul, head_dim, value_dim, key_stride, value_stride,
                      slot_count, start_t, end_t, scale)


def attention_with_sink_into(query, keys, values, sinks, out, heads, kv_mul, head_dim, value_dim, key_stride,
                             value_stride, slot_count, start_t, end_t, scale) -> bool:
    return _attention(query, keys, values, sinks, out, heads, kv_mul, head_dim, value_dim, key_stride, value_stride,
                      slot_count, start_t, end_t, scale)


def attention_noalloc_dev(q_ptr, k_ptr, v_ptr, sinks_ptr, out_ptr, heads, kv_mul, head_dim, value_dim, key_stride,
                          value_stride, slot_count, start_t, end_t, scale) -> bool:
    """rusty_hip_attention_noalloc on device buffers given by address (e.g. a
    torch tensor's data_ptr()); the library allocates nothing for the call."""
    n_kv = heads // kv_mul
    ql, kl, vl = heads * head_dim * 4, slot_count * key_stride * 4, slot_count * value_stride * 4
    ol, sl = heads * value_dim * 4, (heads * 4 if sinks_ptr else 0)
    assert key_stride >= n_kv * head_dim and value_stride >= n_kv * value_dim
    return lib.rusty_hip_attention_noalloc(q_ptr, ql, k_ptr, kl, v_ptr, vl, sinks_ptr or None, sl, out_ptr, ol, heads,
                                           kv_mul, head_dim, value_dim, key_stride, value_stride, slot_count,
                                           start_t, end_t, scale, 1 if sinks_ptr else 0) == 1


# ---- resident decoder (src/metal.rs:302-360) --------------------------------------------
def moe_ffn(x, router, router_dt, router_bias, experts, expert_dt, hidden, biases, top_k):
    """Routed MoE block of gpt-oss decode on the device (rusty_hip_moe_ffn).
    router: bytes [n_experts][dim]; experts = (gate, up, down) expert-major
    block bytes; biases = (gate_b, up_b, down_b) f32 [n_experts][rows] or
    None.  Returns (out, selected experts, weights), or None if unhandled."""
    x = _f32(x)
    dim = x.size
    router = _u8(router)
    n_exp = router.nbytes // (O_ROW_BYTES[router_dt](dim))
    gate, up, down = (_u8(e) for e in experts)
    rb = None if router_bias is None else _f32(router_bias)
    gb, ub, db = (None if b is None else _f32(b) for b in (biases or (None, None, None)))
    out = np.zeros(dim, np.float32)
    sel = np.zeros(top_k, np.int32)
    prob = np.zeros(top_k, np.float32)
    ok = lib.rusty_hip_moe_ffn(_ptr(x), dim, _ptr(router), router.nbytes, router_dt,
                               None if rb is None else _ptr(rb), n_exp, top_k, _ptr(gate), gate.nbytes, _ptr(up),
                               up.nbytes, _ptr(down), down.nbytes, expert_dt, hidden,
                               None if gb is None else _ptr(gb), None if ub is None else _ptr(ub),
                               None if db is None else _ptr(db), _ptr(out), _ptr(sel), _ptr(prob))
    return (out, sel, prob) if ok == 1 else None


O_ROW_BYTES = {8: lambda c: c // 32 * 34, 39: lambda c: c // 32 * 17, 12: lambda c: c // 256 * 144,
               14: lambda c: c // 256 * 210}


class ResidentLayerDesc(C.Structure):
    _fields_ = [("w", C.c_void_p * 7), ("w_len", C.c_size_t * 7), ("w_rows", C.c_uint32 * 7),
                ("w_dt", C.c_uint32 * 7), ("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
                ("bq", C.c_void_p), ("bq_len", C.c_uint32), ("bk", C.c_void_p), ("bk_len", C.c_uint32),
                ("bv", C.c_void_p), ("bv_len", C.c_uint32)]


class Resident:
    """Whole-token-on-device decoder over a model dict from rustyllm_amd.synth."""

    kv_bf16 = False

    def __init__(self, model, storage_len: int, kv_bf16: bool = False):
        cfg = model["config"]
        self.cfg = cfg
        self.storage_len = storage_len
        ok = lib.rusty_hip_resident_configure(cfg["n_layers"], cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"],
                                              cfg["head_dim"], cfg["value_dim"], cfg["hidden_dim"], cfg["vocab"],
                                              storage_len, cfg["eps"], 1 if cfg.get("neox") else 0)
        if ok != 1:
            raise RuntimeError("rusty_hip_resident_configure failed")
        # every host array handed over stays referenced until the call returns
        self._keep = []

        def hold(a, conv):
            a = conv(a)
            self._keep.append(a)
            return _ptr(a)

        for l, layer in enumerate(model["layers"]):
            d = ResidentLayerDesc()
            for i, (arr, dt, rows) in enumerate(layer["w"]):
                d.w[i] = hold(arr, _u8)
                d.w_len[i] = arr.nbytes
                d.w_rows[i] = rows
                d.w_dt[i] = dt
            d.attn_norm = hold(layer["attn_norm"], _f32)
            d.ffn_norm = hold(layer["ffn_norm"], _f32)
            for nm in ("bq", "bk", "bv"):
                b = layer.get(nm)
                if b is not None:
                    setattr(d, nm, hold(b, _f32))
                    setattr(d, nm + "_len", np.asarray(b).size)
            if lib.rusty_hip_resident_set_layer(l, C.byref(d)) != 1:
                raise RuntimeError(f"rusty_hip_resident_set_layer({l}) failed")
        self._set_output(model)
        self._keep = []
        if kv_bf16:
            self.enable_bf16(True)

    def enable_bf16(self, on: bool = True):
        """KVCache::enable_bf16: a fresh bf16 KV cache (kv_read/kv_write then
        move uint16 elements)."""
        if lib.rusty_hip_resident_enable_bf16(1 if on else 0) != 1:
            raise RuntimeError("rusty_hip_resident_enable_bf16 failed")
        self.kv_bf16 = bool(on)

    def _set_output(self, model):
        cfg = self.cfg
        out_w, out_dt = model["output"]
        out_w, inv, norm = _u8(out_w), _f32(model["inv_freq"]), _f32(model["output_norm"])
        if lib.rusty_hip_resident_set_output(_ptr(norm), _ptr(out_w), out_w.nbytes, cfg["vocab"], out_dt, _ptr(inv),
                                             inv.size) != 1:
            raise RuntimeError("rusty_hip_resident_set_output failed")
        emb, emb_dt = model["token_embd"]
        emb = _u8(emb)
        if lib.rusty_hip_resident_set_embedding(_ptr(emb), emb.nbytes, emb_dt) != 1:
            raise RuntimeError("rusty_hip_resident_set_embedding failed")
        self.vocab = cfg["vocab"]

    def decode(self, x_embed, pos, start_t=0, want_logits=True):
        x = _f32(x_embed)
        logits = np.zeros(self.vocab, np.float32)
        ok = lib.rusty_hip_resident_decode(_ptr(x), pos, start_t, 1 if want_logits else 0,
                                           _ptr(logits) if want_logits else None)
        if ok != 1:
            raise RuntimeError("rusty_hip_resident_decode failed")
        return logits

    def prefill(self, tokens, start_pos=0) -> bool:
        """forward_prefill_batch: KV cache over tokens at start_pos.. (no
        logits).  False when the model is not batchable."""
        t = np.ascontiguousarray(tokens, np.int32)
        return lib.rusty_hip_resident_prefill(_ptr(t), t.size, start_pos) == 1

    def generate(self, prompt, n_gen, penalty=1.1, start_pos=0, want_logits=True):
        p = np.ascontiguousarray(prompt, np.int32)
        toks = np.zeros(max(n_gen, 1), np.int32)
        logits = np.zeros(self.vocab, np.float32)
        ok = lib.rusty_hip_resident_generate(_ptr(p), p.size, start_pos, n_gen, penalty, _ptr(toks),
                                             _ptr(logits) if want_logits else None)
        if ok != 1:
            raise RuntimeError("rusty_hip_resident_generate failed")
        return toks[:n_gen], logits

    def kv_read(self, layer, which, slot0, n_slots):
        cfg = self.cfg
        w = cfg["n_kv_heads"] * (cfg["value_dim"] if which else cfg["head_dim"])
        out = np.zeros(n_slots * w, np.uint16 if self.kv_bf16 else np.float32)
        if lib.rusty_hip_resident_kv_read(layer, which, slot0, n_slots, _ptr(out)) != 1:
            raise RuntimeError("kv_read failed")
        return out

    def kv_write(self, layer, which, slot0, data):
        cfg = self.cfg
        w = cfg["n_kv_heads"] * (cfg["value_dim"] if which else cfg["head_dim"])
        d = np.ascontiguousarray(data, np.uint16) if self.kv_bf16 else _f32(data)
        n_slots = d.size // w
        if lib.rusty_hip_resident_kv_write(layer, which, slot0, n_slots, _ptr(d)) != 1:
            raise RuntimeError("kv_write failed")

    def time_decode(self, n_tokens, penalty=1.1) -> float:
        ms = C.c_double(0.0)
        if lib.rusty_hip_resident_time_decode(n_tokens, penalty, C.byref(ms)) != 1:
            raise RuntimeError("rusty_hip_resident_time_decode failed")
        return ms.value


class MoeLayerDesc(C.Structure):
    _fields_ = [("w", C.c_void_p * 4), ("w_len", C.c_size_t * 4), ("w_dt", C.c_uint32 * 4),
                ("bq", C.c_void_p), ("bk", C.c_void_p), ("bv", C.c_void_p), ("bo", C.c_void_p),
                ("sinks", C.c_void_p), ("attn_norm", C.c_void_p), ("post_attn_norm", C.c_void_p),
                ("router", C.c_void_p), ("router_len", C.c_size_t), ("router_dt", C.c_uint32),
                ("router_bias", C.c_void_p), ("exps", C.c_void_p * 3), ("exps_len", C.c_size_t * 3),
                ("exps_dt", C.c_uint32), ("exps_bias", C.c_void_p * 3)]


class ResidentGptOss(Resident):
    """The resident decoder in gpt-oss mode over a model from
    rustyllm_amd.synth.make_gptoss (rusty_hip_resident_configure_moe)."""

    def __init__(self, model, max_len: int):
        """max_len: positions the cache holds (the reference's KVCache
        max_len); with a sliding window the device keeps a ring of
        min(window, max_len) slots."""
        cfg = self.cfg = model["config"]
        self.storage_len = max_len
        w = cfg.get("window", 0)
        self.slots = min(w, max_len) if w > 0 else max_len
        self._keep = []

        def hold(a, conv):
            a = conv(a)
            self._keep.append(a)
            return _ptr(a)

        ok = lib.rusty_hip_resident_configure_moe(cfg["n_layers"], cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"],
                                                  cfg["head_dim"], cfg["hidden_dim"], cfg["n_experts"],
                                                  cfg["top_k"], cfg["vocab"], max_len, w, cfg["eps"],
                                                  model["concentration"])
        if ok != 1:
            raise RuntimeError("rusty_hip_resident_configure_moe failed")
        router_dt = model.get("router_type", Q8_0)
        exps_dt = model.get("experts_type", MXFP4)
        for l, L in enumerate(model["layers"]):
            d = MoeLayerDesc()
            for i, nm in enumerate(("wq", "wk", "wv", "wo")):
                arr, t = L[nm]
                d.w[i], d.w_len[i], d.w_dt[i] = hold(arr, _u8), arr.nbytes, t
            for nm in ("bq", "bk", "bv", "bo", "sinks", "attn_norm", "post_attn_norm", "router_bias"):
                setattr(d, nm, hold(L[nm], _f32))
            d.router, d.router_len, d.router_dt = hold(L["router"], _u8), L["router"].nbytes, router_dt
            for i, nm in enumerate(("gate_exps", "up_exps", "down_exps")):
                d.exps[i], d.exps_len[i] = hold(L[nm], _u8), L[nm].nbytes
                d.exps_bias[i] = hold(L[nm + "_bias"], _f32)
            d.exps_dt = exps_dt
            if lib.rusty_hip_resident_set_moe_layer(l, C.byref(d)) != 1:
                raise RuntimeError(f"rusty_hip_resident_set_moe_layer({l}) failed")
        self._set_output(model)
        self._keep = []


class ResidentGguf(Resident):
    """The resident decoder configured straight from a GGUF file by the
    library (rusty_hip_resident_load_gguf): mapped, parsed and uploaded
    natively, no host model in between."""

    def __init__(self, path: str, max_len: int):
        s = gguf_summary(path)
        if s is None:
            raise RuntimeError(f"{path}: not a readable GGUF file")
        if lib.rusty_hip_resident_load_gguf(os.fsencode(path), max_len) != 1:
            raise RuntimeError(f"rusty_hip_resident_load_gguf({path}) failed")
        self.summary = s
        self.cfg = {"n_kv_heads": s.n_kv_heads, "head_dim": s.head_dim, "value_dim": s.value_dim,
                    "n_layers": s.n_layers, "dim": s.dim}
        self.storage_len = max_len
        self.vocab = s.vocab


# ---- profiling -------------------------------------------------------------------------
def profile_enable(on: bool) -> None:
    lib.rusty_hip_profile_enable(1 if on else 0)


def profile_results():
    out = {}
    i = 0
    name = C.create_string_buffer(64)
    tot = C.c_double(0)
    cnt = C.c_int64(0)
    while lib.rusty_hip_profile_get(i, name, C.byref(tot), C.byref(cnt)) == 1:
        out[name.value.decode()] = (tot.value, cnt.value)
        i += 1
    return out


def bench_matvec(ggml_type: int, weights: np.ndarray, x: np.ndarray, rows: int, cols: int, copies: int,
                 iters: int) -> np.ndarray:
    """iters device-resident GEMV launches over `copies` rotated weight copies
    (kernel sweep); returns the last output.  Durations land in the profile."""
    w, x = _u8(weights), _f32(x)
    out = np.empty(rows, np.float32)
    if lib.rusty_hip_bench_matvec(ggml_type, _ptr(w), w.nbytes, _ptr(x), rows, cols, copies, iters, _ptr(out)) != 1:
        raise RuntimeError("rusty_hip_bench_matvec failed")
    return out


def bench_attention(heads: int, kv_mul: int, head_dim: int, ctx: int, copies: int, iters: int, seed: int,
                    mode: str = "exact") -> np.ndarray:
    """iters decode-attention launches over `copies` rotated device K/V sets
    of ctx positions (kernel sweep); returns the last output."""
    out = np.empty(heads * head_dim, np.float32)
    code = {"exact": 0, "fast": 1}[mode]
    if lib.rusty_hip_bench_attention(heads, kv_mul, head_dim, ctx, copies, iters, seed, code, _ptr(out)) != 1:
        raise RuntimeError("rusty_hip_bench_attention failed")
    return out


def sync() -> None:
    lib.rusty_hip_sync()


def attention_mode(mode: str | None = None) -> str:
    """'exact' (reference order, bit for bit; default) or 'fast' (split-K).
    Returns the mode in force before the call."""
    code = {"exact": 0, "fast": 1, None: -1}[mode]
    return "fast" if lib.rusty_hip_attention_mode(code) == 1 else "exact"


def debug_expf(x):
    x = _f32(x)
    out = np.zeros_like(x)
    assert lib.rusty_hip_debug_expf(_ptr(x), x.size, _ptr(out)) == 1
    return out


def weight_cache_clear() -> None:
    """Drops device copies cached by host address (call before host weight
    arrays are freed and their memory may be reused)."""
    lib.rusty_hip_weight_cache_clear()


# ---- debug hooks ----------------------------------------------------------------------
def debug_quantize_q8k(x):
    x = _f32(x)
    n = x.size
    qs = np.zeros(n, np.int8)
    d = np.zeros(n // 256, np.float32)
    bs = np.zeros(n // 32, np.int16)
    assert lib.rusty_hip_debug_quantize_q8k(_ptr(x), n, _ptr(qs), _ptr(d), _ptr(bs)) == 1
    return qs, d, bs


def debug_dequant(ggml_type, w, rows, cols):
    w = _u8(w)
    out = np.zeros(rows * cols, np.float32)
    assert lib.rusty_hip_debug_dequant(ggml_type, _ptr(w), w.nbytes, rows, cols, _ptr(out)) == 1
    return out.reshape(rows, cols)


def debug_block_ints(ggml_type, w, rows, cols, x):
    w, x = _u8(w), _f32(x)
    if ggml_type == Q8_0:
        n = rows * (cols // 32)
    elif ggml_type == Q4_K:
        n = rows * (cols // 256) * 2
    else:
        n = rows * (cols // 256)
    out = np.zeros(n, np.int32)
    assert lib.rusty_hip_debug_block_ints(ggml_type, _ptr(w), w.nbytes, rows, cols, _ptr(x), _ptr(out)) == 1
    return out


def debug_rmsnorm(x, w, eps):
    x, w = _f32(x), _f32(w)
    out = np.zeros_like(x)
    assert lib.rusty_hip_debug_rmsnorm(_ptr(x), _ptr(w), eps, x.size, _ptr(out)) == 1
    return out


def debug_silu_mul(g_, u):
    g_, u = _f32(g_), _f32(u)
    out = np.zeros_like(g_)
    assert lib.rusty_hip_debug_silu_mul(_ptr(g_), _ptr(u), g_.size, _ptr(out)) == 1
    return out


def debug_rope(q, k, pos, head_dim, n_heads, n_kv, inv_freq, neox=False):
    q, k, inv = _f32(q).copy(), _f32(k).copy(), _f32(inv_freq)
    assert lib.rusty_hip_debug_rope(_ptr(q), _ptr(k), pos, head_dim, n_heads, n_kv, _ptr(inv), 1 if neox else 0) == 1
    return q, k


def debug_greedy(logits, recent, penalty):
    lg = _f32(logits)
    r = np.ascontiguousarray(recent, np.int32)
    tok = C.c_int32(0)
    assert lib.rusty_hip_debug_greedy(_ptr(lg), lg.size, _ptr(r) if r.size else None, r.size, penalty,
                                      C.byref(tok)) == 1
    return tok.value


def debug_f16(h):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.zeros(h.size, np.float32)
    assert lib.rusty_hip_debug_f16(_ptr(h), h.size, _ptr(out)) == 1
    return out


def debug_stream_mark() -> bool:
    """Marks the resident decoder's next streamed attention launch as timed
    out (the failure path's test hook)."""
    return lib.rusty_hip_debug_stream_mark() == 1


def set_expert_mfma(on: bool) -> bool:
    """rusty_hip_set_expert_mfma: the gpt-oss prefill's expert product on the
    matrix cores (True) or as the reference's serial sums (False, the
    default).  Returns the previous setting."""
    return lib.rusty_hip_set_expert_mfma(1 if on else 0) == 1


def mxfp4_experts_dev(w_ptr, row_stride, exp_stride, n_exp, rows, cols, x_ptr, ldx, x_per_pair, top_k, sel_ptr,
                      n_pairs, y_ptr, ldy, mfma) -> bool:
    """rusty_hip_mxfp4_experts on device buffers given by address."""
    return lib.rusty_hip_mxfp4_experts(w_ptr, row_stride, exp_stride, n_exp, rows, cols, x_ptr, ldx,
                                       1 if x_per_pair else 0, top_k, sel_ptr, n_pairs, y_ptr, ldy,
                                       1 if mfma else 0) == 1
