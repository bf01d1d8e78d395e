"""ctypes bindings for the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the CPU
baseline that bench.py reports.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module.  It restates
SimonWaldherr/RustyLLM's x86-64 numerics (src/simd.rs, src/model.rs); each C
function cites the reference line it follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, Q8_0, Q4_K, Q6_K, MXFP4 = 0, 8, 12, 14, 39
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), MXFP4: (32, 17), F32: (1, 4)}


def build() -> None:
    """Compile liboracle.so from oracle.c (make, in this directory)."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)


def _load() -> C.CDLL:
    if not os.path.exists(_LIB_PATH):
        build()
    return C.CDLL(_LIB_PATH)


lib = _load()
_p = C.c_void_p
_i64 = C.c_int64
_f = C.c_float


def _sig(name, res, *args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = list(args)
    return fn


_sig("orc_f16_to_f32", _f, C.c_uint16)
_sig("orc_mxfp4_scale", _f, C.c_uint8)
_sig("orc_quantize_row_q8k_scalar", None, _p, _i64, _p, _p, _p)
_sig("orc_quantize_row_q8k_avx2", None, _p, _i64, _p, _p, _p)
_sig("orc_dequant_row", None, C.c_int, _p, _p, _i64)
for _n in ("orc_dot_q4_k_q8k_avx2", "orc_dot_q6_k_q8k_avx2", "orc_dot_q8_0_q8k_avx2", "orc_emulate_q4_k_q8k"):
    _sig(_n, _f, _p, _p, _p, _p, _i64)
_sig("orc_emulate_q6_k_q8k", _f, _p, _p, _p, _i64)
_sig("orc_emulate_q8_0_q8k", _f, _p, _p, _p, _i64)
_sig("orc_dot_q8_0_f32_avx2", _f, _p, _p, _i64)
_sig("orc_dot_mxfp4_f32_scalar", _f, _p, _p, _i64)
_sig("orc_dot_f32_avx2", _f, _p, _p, _i64)
_sig("orc_q4k_block_ints", None, _p, _p, _p, _i64, _p, _p)
_sig("orc_q6k_block_ints", None, _p, _p, _i64, _p)
_sig("orc_q8_0_block_ints", None, _p, _p, _i64, _p)
_sig("orc_row_bytes", _i64, C.c_int, _i64)
_sig("orc_matvec", None, C.c_int, _p, _p, _i64, _i64, _p, C.c_int)
_sig("orc_set_threads", None, C.c_int)
_sig("orc_set_fast_schedule", None, C.c_int)
_sig("orc_online_attention", None, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f, _p)
_sig("orc_online_attention_with_sink", None, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f, _f, _p)
_sig("orc_online_attention_grouped", None, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f, _p)
_sig("orc_attention_over_kv_heads", None, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f, _p)
_sig("orc_attention_sink_heads", None, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f, _p)
_sig("orc_attention_start_pos", _i64, _i64, _i64)
_sig("orc_f32_to_bf16", C.c_uint16, _f)
_sig("orc_bf16_to_f32", _f, C.c_uint16)
_sig("orc_dot_bf16_f32_avx2", _f, _p, _p, _i64)
_sig("orc_attention_over_kv_heads_bf16", None, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f,
     _p)
_sig("orc_rms_norm", None, _p, _p, _f, _i64, _p)
_sig("orc_build_rope_inv_freq", None, _f, _i64, _f, _p)
_sig("orc_rope_qk", None, _p, _p, _i64, _i64, _i64, _i64, _p)
_sig("orc_rope_qk_neox", None, _p, _p, _i64, _i64, _i64, _i64, _p)
_sig("orc_rope_gpt_oss", None, _p, _p, _i64, _i64, _i64, _i64, _f, _p)
_sig("orc_build_rope_inv_freq_gpt_oss", None, _f, _i64, _f, _i64, _p, _p)
_sig("orc_silu_mul_avx2", None, _p, _p, _p, _i64)
_sig("orc_silu_mul_scalar", None, _p, _p, _p, _i64)
_sig("orc_swiglu_gpt_oss", _f, _f, _f)
_sig("orc_select_top_logits", None, _p, _i64, _i64, _p, _p)
_sig("orc_softmax_selected", None, _p, _i64, _p)
_sig("orc_apply_repeat_penalty", None, _p, _i64, _p, _i64, _f)
_sig("orc_argmax_finite", C.c_uint32, _p, _i64)
_sig("orc_greedy", C.c_uint32, _p, _i64, _p, _i64, _f)
_sig("orc_expf_array", None, _p, _i64, _p)
_sig("orc_model_create", _p, _p)
_sig("orc_model_free", None, _p)
_sig("orc_model_set_layer", C.c_int, _p, C.c_int32, _p)
_sig("orc_model_set_output", C.c_int, _p, _p, _p, C.c_uint32, _p, C.c_uint32, _p)
_sig("orc_model_forward", None, _p, C.c_uint32, _i64, _p, C.c_int)
_sig("orc_model_forward_from", None, _p, C.c_uint32, _i64, _i64, _p, C.c_int)
_sig("orc_model_kv", C.POINTER(C.c_float), _p, C.c_int32, C.c_int32)
_sig("orc_model_generate", _i64, _p, _p, _i64, _i64, _i64, _f, _p, _p)
_sig("orc_gptoss_create", _p, _p)
_sig("orc_gptoss_free", None, _p)
_sig("orc_gptoss_set_layer", C.c_int, _p, C.c_int32, _p)
_sig("orc_gptoss_set_output", C.c_int, _p, _p, _p, C.c_uint32, _p, C.c_uint32, _p)
_sig("orc_gptoss_storage", _i64, _p)
_sig("orc_gptoss_kv", C.POINTER(C.c_float), _p, C.c_int32, C.c_int32)
_sig("orc_gptoss_forward", None, _p, C.c_uint32, _i64, _p, C.c_int)
_sig("orc_make_q4k_weights", None, _i64, _i64, C.c_uint8, _p)
_sig("orc_make_q4k_weights_dmin", None, _i64, _i64, C.c_uint8, _p)
_sig("orc_make_q6k_weights", None, _i64, _i64, C.c_uint8, _p)
_sig("orc_make_q8_0_row_scaled", None, _i64, C.c_uint8, _p)
_sig("orc_make_mxfp4_test_row", None, _i64, _p)
_sig("orc_test_activation", None, _i64, _p)
_sig("orc_mxfp4_test_activation", None, _i64, _p)


def ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def row_bytes(dtype: int, cols: int) -> int:
    return int(lib.orc_row_bytes(dtype, cols))


# ---- Q8_K ------------------------------------------------------------------
def quantize_q8k(x: np.ndarray, avx2: bool = True):
    x = f32(x)
    n = x.size
    qs = np.zeros(n, np.int8)
    d = np.zeros(n // 256, np.float32)
    bs = np.zeros(n // 32, np.int16)
    fn = lib.orc_quantize_row_q8k_avx2 if avx2 else lib.orc_quantize_row_q8k_scalar
    fn(ptr(x), n, ptr(qs), ptr(d), ptr(bs))
    return qs, d, bs


def dequant_row(dtype: int, q: np.ndarray, n: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    out = np.empty(n, np.float32)
    lib.orc_dequant_row(dtype, ptr(q), ptr(out), n)
    return out


def dequant(dtype: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    rb = row_bytes(dtype, cols)
    out = np.empty((rows, cols), np.float32)
    for r in range(rows):
        lib.orc_dequant_row(dtype, ptr(w) + r * rb, ptr(out) + r * cols * 4, cols)
    return out


def matvec(dtype: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int, threads: int = 0) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    x = f32(x)
    out = np.empty(rows, np.float32)
    lib.orc_matvec(dtype, ptr(w), ptr(x), rows, cols, ptr(out), threads)
    return out


def block_ints(dtype: int, w_row: np.ndarray, qs: np.ndarray, bs: np.ndarray, cols: int):
    w_row = np.ascontiguousarray(w_row, np.uint8)
    if dtype == Q4_K:
        isum = np.zeros(cols // 256, np.int32)
        imin = np.zeros(cols // 256, np.int32)
        lib.orc_q4k_block_ints(ptr(w_row), ptr(qs), ptr(bs), cols, ptr(isum), ptr(imin))
        return isum, imin
    if dtype == Q6_K:
        isum = np.zeros(cols // 256, np.int32)
        lib.orc_q6k_block_ints(ptr(w_row), ptr(qs), cols, ptr(isum))
        return isum, None
    if dtype == Q8_0:
        s = np.zeros(cols // 32, np.int32)
        lib.orc_q8_0_block_ints(ptr(w_row), ptr(qs), cols, ptr(s))
        return s, None
    raise ValueError(dtype)


def attention(q, k, v, n_heads, n_kv, hd, vd, key_stride, value_stride, slot_count, start_t, end_t, scale,
              sinks=None) -> np.ndarray:
    """Reference attention over all heads: grouped GQA (model.rs:5952) or, with
    sinks, the gpt-oss per-head sink loop (model.rs:6812-6833)."""
    q, k, v = f32(q), f32(k), f32(v)
    out = np.zeros(n_heads * vd, np.float32)
    kv_mul = n_heads // n_kv
    if sinks is None:
        lib.orc_attention_over_kv_heads(ptr(q), ptr(k), ptr(v), key_stride, value_stride, slot_count, hd, vd,
                                        n_kv, kv_mul, start_t, end_t, scale, ptr(out))
    else:
        s = f32(sinks)
        lib.orc_attention_sink_heads(ptr(q), ptr(k), ptr(v), ptr(s), key_stride, value_stride, slot_count, hd, vd,
                                     n_heads, kv_mul, start_t, end_t, scale, ptr(out))
    return out


def f32_to_bf16(x) -> np.ndarray:
    """f32_to_bf16 (simd.rs:88-96) per element: uint16 bit patterns."""
    x = f32(x).reshape(-1)
    return np.array([lib.orc_f32_to_bf16(float(v)) for v in x], np.uint16)


def attention_bf16(q, k16, v16, n_heads, n_kv, hd, vd, key_stride, value_stride, slot_count, start_t, end_t,
                   scale) -> np.ndarray:
    """attention_over_kv_heads_bf16 (model.rs:6508-6580) over uint16 bf16 K/V."""
    q = f32(q)
    k16, v16 = np.ascontiguousarray(k16, np.uint16), np.ascontiguousarray(v16, np.uint16)
    out = np.zeros(n_heads * vd, np.float32)
    lib.orc_attention_over_kv_heads_bf16(ptr(q), ptr(k16), ptr(v16), key_stride, value_stride, slot_count, hd, vd,
                                         n_kv, n_heads // n_kv, start_t, end_t, scale, ptr(out))
    return out


def rms_norm(x, w, eps):
    x, w = f32(x), f32(w)
    out = np.empty_like(x)
    lib.orc_rms_norm(ptr(x), ptr(w), eps, x.size, ptr(out))
    return out


def rope_inv_freq(theta: float, head_dim: int, scaling: float = 1.0) -> np.ndarray:
    inv = np.zeros(head_dim // 2, np.float32)
    lib.orc_build_rope_inv_freq(theta, head_dim, scaling, ptr(inv))
    return inv


def rope(q, k, pos, hd, nh, nkv, inv_freq, neox=False):
    q, k, inv = f32(q).copy(), f32(k).copy(), f32(inv_freq)
    (lib.orc_rope_qk_neox if neox else lib.orc_rope_qk)(ptr(q), ptr(k), pos, hd, nh, nkv, ptr(inv))
    return q, k


def silu_mul(gate, up, avx2=True):
    g, u = f32(gate), f32(up)
    out = np.empty_like(g)
    (lib.orc_silu_mul_avx2 if avx2 else lib.orc_silu_mul_scalar)(ptr(g), ptr(u), ptr(out), g.size)
    return out


def greedy(logits, recent, penalty):
    lg = f32(logits).copy()
    r = np.ascontiguousarray(recent, np.uint32)
    tok = lib.orc_greedy(ptr(lg), lg.size, ptr(r) if r.size else None, r.size, penalty)
    return int(tok), lg


def expf(x):
    x = f32(x)
    out = np.empty_like(x)
    lib.orc_expf_array(ptr(x), x.size, ptr(out))
    return out


def top_k_router(logits, k):
    lg = f32(logits)
    idx = np.zeros(k, np.int32)
    val = np.zeros(k, np.float32)
    lib.orc_select_top_logits(ptr(lg), lg.size, k, ptr(idx), ptr(val))
    probs = np.zeros(k, np.float32)
    lib.orc_softmax_selected(ptr(val), k, ptr(probs))
    return idx, val, probs


def rope_inv_freq_gpt_oss(theta: float, head_dim: int, scaling: float, orig_ctx: int):
    """build_rope_inv_freq_gpt_oss (model.rs:3059-3098): (inv_freq, concentration)."""
    inv = np.zeros(head_dim // 2, np.float32)
    conc = C.c_float(0.0)
    lib.orc_build_rope_inv_freq_gpt_oss(theta, head_dim, scaling, orig_ctx, ptr(inv), C.addressof(conc))
    return inv, float(conc.value)


def rope_gpt_oss(q, k, pos, hd, nh, nkv, concentration, inv_freq):
    q, k, inv = f32(q).copy(), f32(k).copy(), f32(inv_freq)
    lib.orc_rope_gpt_oss(ptr(q), ptr(k), pos, hd, nh, nkv, concentration, ptr(inv))
    return q, k


def swiglu_gpt_oss(g, u):
    return np.array([lib.orc_swiglu_gpt_oss(float(a), float(b)) for a, b in zip(g, u)], np.float32)


def moe_block(x, router, router_t, router_bias, experts, experts_t, hidden, biases, top_k):
    """Routed MoE block of forward_gpt_oss_into (model.rs:6846-6898): router
    matvec + bias, top-k in total order (select_top_logits_into), softmax over
    the chosen (softmax_selected_into), per expert swiglu_gpt_oss of gate/up
    (+ biases), down (+ bias), weighted sum in slot order.  Returns (moe,
    selected experts, weights)."""
    x = f32(x)
    dim = x.size
    n_exp = router.nbytes // row_bytes(router_t, dim)
    logits = matvec(router_t, router, x, n_exp, dim)
    if router_bias is not None:
        logits = (logits + router_bias).astype(np.float32)
    idx, _, probs = top_k_router(logits, top_k)
    gate, up, down = experts
    gb, ub, db = biases if biases is not None else (None, None, None)
    rg, rd = row_bytes(experts_t, dim) * hidden, row_bytes(experts_t, hidden) * dim
    moe = np.zeros(dim, np.float32)
    for s, e in enumerate(idx):
        g = matvec(experts_t, gate[e * rg:(e + 1) * rg], x, hidden, dim)
        u = matvec(experts_t, up[e * rg:(e + 1) * rg], x, hidden, dim)
        if gb is not None:
            g = (g + gb[e]).astype(np.float32)
        if ub is not None:
            u = (u + ub[e]).astype(np.float32)
        d = matvec(experts_t, down[e * rd:(e + 1) * rd], swiglu_gpt_oss(g, u), dim, hidden)
        if db is not None:
            d = (d + db[e]).astype(np.float32)
        moe = (moe + d * probs[s]).astype(np.float32)
    return moe, idx, probs


class OracleGptOssComposed:
    """forward_gpt_oss_into (model.rs:6733-6908) composed in Python from the
    C restatements of its parts, with the KV cache on the host; it checks the
    C layer loop (OracleGptOss) step for step on small models.  The cache is the
    reference's KVCache::with_sliding_window(max_len, window)
    (model.rs:1363-1385): with a window it is a ring of
    storage_len_for(max_len, window) = min(window, max_len) slots and
    position p lives in slot p % storage (slot_for_pos, :1458-1464); every
    layer's attention scans that ring with slot_count = storage
    (:6793-6810), the full (odd) layers from position 0.  Test infrastructure
    only."""

    def __init__(self, model, max_len: int):
        self.m = model
        c = self.c = model["config"]
        self.max_len = max(1, max_len)
        w = c.get("window", 0)
        self.storage = min(w, self.max_len) if w > 0 else self.max_len
        self.ring = w > 0
        self.kd = c["n_kv_heads"] * c["head_dim"]
        self.vdim = c["n_kv_heads"] * c["value_dim"]
        self.kc = [np.zeros(self.storage * self.kd, np.float32) for _ in model["layers"]]
        self.vc = [np.zeros(self.storage * self.vdim, np.float32) for _ in model["layers"]]

    def slot(self, pos: int) -> int:
        return pos % self.storage if self.ring else pos

    def forward(self, token: int, pos: int) -> np.ndarray:
        m, c = self.m, self.c
        dim, nh, nkv, hd, vd = c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["value_dim"]
        emb, emb_t = m["token_embd"]
        x = dequant_row(emb_t, emb[token * row_bytes(emb_t, dim):], dim)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        for l, L in enumerate(m["layers"]):
            xn = rms_norm(x, L["attn_norm"], c["eps"])
            q = (matvec(L["wq"][1], L["wq"][0], xn, nh * hd, dim) + L["bq"]).astype(np.float32)
            k = (matvec(L["wk"][1], L["wk"][0], xn, nkv * hd, dim) + L["bk"]).astype(np.float32)
            v = (matvec(L["wv"][1], L["wv"][0], xn, nkv * vd, dim) + L["bv"]).astype(np.float32)
            q, k = rope_gpt_oss(q, k, pos, hd, nh, nkv, m["concentration"], m["inv_freq"])
            sl = self.slot(pos)
            self.kc[l][sl * self.kd:(sl + 1) * self.kd] = k
            self.vc[l][sl * self.vdim:(sl + 1) * self.vdim] = v
            start = int(lib.orc_attention_start_pos(pos, c["window"])) if l % 2 == 0 else 0
            attn = attention(q, self.kc[l], self.vc[l], nh, nkv, hd, vd, self.kd, self.vdim, self.storage, start,
                             pos, scale, sinks=L["sinks"])
            proj = matvec(L["wo"][1], L["wo"][0], attn, dim, nh * vd)
            x = (x + (proj + L["bo"]).astype(np.float32)).astype(np.float32)
            xn2 = rms_norm(x, L["post_attn_norm"], c["eps"])
            moe, _, _ = moe_block(xn2, L["router"], Q8_0, L["router_bias"],
                                  (L["gate_exps"], L["up_exps"], L["down_exps"]), MXFP4, c["hidden_dim"],
                                  (L["gate_exps_bias"], L["up_exps_bias"], L["down_exps_bias"]), c["top_k"])
            x = (x + moe).astype(np.float32)
        xn = rms_norm(x, m["output_norm"], c["eps"])
        out, out_t = m["output"]
        return matvec(out_t, out, xn, c["vocab"], dim)

    def generate(self, prompt, n_gen, penalty=1.1, start_pos=0):
        """The decode loop of the reference runtime (greedy + repeat penalty
        over the last <= 64 tokens, runtime.rs:493-521), as orc_model_generate."""
        recent = [int(t) for t in prompt[-64:]]
        pos = start_pos
        logits = None
        for i, t in enumerate(prompt):
            logits = self.forward(int(t), pos)
            pos += 1
        toks = []
        for g in range(n_gen):
            last = logits
            tok, _ = greedy(logits, recent, penalty)
            toks.append(tok)
            recent = (recent + [tok])[-64:]
            if g + 1 == n_gen:
                break
            logits = self.forward(tok, pos)
            pos += 1
        return np.array(toks, np.uint32), last


class OrcGptOssConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "value_dim",
                                          "hidden_dim", "n_experts", "top_k", "vocab", "max_len", "sliding_window")] + \
               [("eps", C.c_float), ("concentration", C.c_float)]


class OrcGptOssLayer(C.Structure):
    _fields_ = [("wq", _p), ("wk", _p), ("wv", _p), ("wo", _p), ("wq_type", C.c_uint32), ("wk_type", C.c_uint32),
                ("wv_type", C.c_uint32), ("wo_type", C.c_uint32)] + \
               [(n, _p) for n in ("bq", "bk", "bv", "bo", "sinks", "attn_norm", "post_attn_norm", "router")] + \
               [("router_type", C.c_uint32), ("router_bias", _p), ("gate_exps", _p), ("up_exps", _p),
                ("down_exps", _p), ("exps_type", C.c_uint32), ("gate_exps_bias", _p), ("up_exps_bias", _p),
                ("down_exps_bias", _p)]


class OracleGptOss:
    """forward_gpt_oss_into (model.rs:6733-6908) as one C layer loop
    (orc_gptoss_forward), with the reference's window-sized ring KV cache
    (KVCache::with_sliding_window, model.rs:1363-1385): storage =
    min(window, max_len) slots, position p at slot p % storage, every layer's
    attention over that ring, the odd (full) layers from position 0.
    forward(..., want_logits=False) is forward_prefill_gpt_oss (no head).
    kc[l] / vc[l] are numpy views of the C cache (writes reach the oracle).
    Test infrastructure only."""

    def __init__(self, model, max_len: int, threads: int = 0):
        self.m = model
        c = self.c = model["config"]
        self.max_len = max(1, max_len)
        w = c.get("window", 0)
        self.ring = w > 0
        cfg = OrcGptOssConfig(c["n_layers"], c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["value_dim"],
                              c["hidden_dim"], c["n_experts"], c["top_k"], c["vocab"], self.max_len, w, c["eps"],
                              model["concentration"])
        if threads:
            lib.orc_set_threads(threads)
        self.h = lib.orc_gptoss_create(C.byref(cfg))
        self.storage = int(lib.orc_gptoss_storage(self.h))
        self._keep = []

        def hold(a, dt=np.float32):
            a = np.ascontiguousarray(a, dt)
            self._keep.append(a)
            return ptr(a)

        for l, L in enumerate(model["layers"]):
            d = OrcGptOssLayer()
            for nm in ("wq", "wk", "wv", "wo"):
                setattr(d, nm, hold(L[nm][0], np.uint8))
                setattr(d, nm + "_type", L[nm][1])
            for nm in ("bq", "bk", "bv", "bo", "sinks", "attn_norm", "post_attn_norm", "router_bias",
                       "gate_exps_bias", "up_exps_bias", "down_exps_bias"):
                setattr(d, nm, hold(L[nm]))
            d.router, d.router_type = hold(L["router"], np.uint8), Q8_0
            for nm in ("gate_exps", "up_exps", "down_exps"):
                setattr(d, nm, hold(L[nm], np.uint8))
            d.exps_type = MXFP4
            lib.orc_gptoss_set_layer(self.h, l, C.byref(d))
        out_w, out_t = model["output"]
        emb, emb_t = model["token_embd"]
        lib.orc_gptoss_set_output(self.h, hold(model["output_norm"]), hold(out_w, np.uint8), out_t,
                                  hold(emb, np.uint8), emb_t, hold(model["inv_freq"]))
        kd = c["n_kv_heads"] * c["head_dim"]
        vdim = c["n_kv_heads"] * c["value_dim"]
        self.kc = [np.ctypeslib.as_array(lib.orc_gptoss_kv(self.h, l, 0), shape=(self.storage * kd,))
                   for l in range(c["n_layers"])]
        self.vc = [np.ctypeslib.as_array(lib.orc_gptoss_kv(self.h, l, 1), shape=(self.storage * vdim,))
                   for l in range(c["n_layers"])]

    def slot(self, pos: int) -> int:
        return pos % self.storage if self.ring else pos

    def forward(self, token: int, pos: int, want_logits: bool = True) -> np.ndarray:
        logits = np.zeros(self.c["vocab"], np.float32)
        lib.orc_gptoss_forward(self.h, int(token), int(pos), ptr(logits), 1 if want_logits else 0)
        return logits

    def generate(self, prompt, n_gen, penalty=1.1, start_pos=0):
        """The decode loop of the reference runtime (forward_prefill_gpt_oss
        per prompt token but the last, runtime.rs:3760-3790; greedy + repeat
        penalty over the last <= 64 tokens, runtime.rs:493-521)."""
        recent = [int(t) for t in prompt[-64:]]
        pos = start_pos
        logits = None
        for i, t in enumerate(prompt):
            logits = self.forward(int(t), pos, want_logits=i + 1 == len(prompt))
            pos += 1
        toks = []
        last = logits
        for g in range(n_gen):
            last = logits
            tok, _ = greedy(logits, recent, penalty)
            toks.append(tok)
            recent = (recent + [tok])[-64:]
            if g + 1 == n_gen:
                break
            logits = self.forward(tok, pos)
            pos += 1
        return np.array(toks, np.uint32), last

    def __del__(self):
        try:
            lib.orc_gptoss_free(self.h)
        except Exception:
            pass


# ---- reference fixtures ------------------------------------------------------
def make_q4k_weights(rows, cols, seed, dmin=False):
    out = np.zeros(rows * (cols // 256) * 144, np.uint8)
    (lib.orc_make_q4k_weights_dmin if dmin else lib.orc_make_q4k_weights)(rows, cols, seed, ptr(out))
    return out


def make_q6k_weights(rows, cols, seed):
    out = np.zeros(rows * (cols // 256) * 210, np.uint8)
    lib.orc_make_q6k_weights(rows, cols, seed, ptr(out))
    return out


def make_q8_0_row_scaled(cols, seed):
    out = np.zeros((cols // 32) * 34, np.uint8)
    lib.orc_make_q8_0_row_scaled(cols, seed, ptr(out))
    return out


def make_mxfp4_test_row(blocks):
    out = np.zeros(blocks * 17, np.uint8)
    lib.orc_make_mxfp4_test_row(blocks, ptr(out))
    return out


def test_activation(cols):
    out = np.zeros(cols, np.float32)
    lib.orc_test_activation(cols, ptr(out))
    return out


def mxfp4_test_activation(n):
    out = np.zeros(n, np.float32)
    lib.orc_mxfp4_test_activation(n, ptr(out))
    return out


# ---- model -------------------------------------------------------------------
class OrcConfig(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("dim", C.c_int32), ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32),
                ("head_dim", C.c_int32), ("value_dim", C.c_int32), ("hidden_dim", C.c_int32), ("vocab", C.c_int32),
                ("storage_len", C.c_int32), ("sliding_window", C.c_int32), ("neox", C.c_int32), ("eps", C.c_float),
                ("kv_bf16", C.c_int32)]


class OrcLayer(C.Structure):
    _fields_ = [("w", C.c_void_p * 7), ("w_len", C.c_uint64 * 7), ("w_rows", C.c_uint32 * 7),
                ("w_type", C.c_uint32 * 7), ("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
                ("bq", C.c_void_p), ("bq_len", C.c_uint32), ("bk", C.c_void_p), ("bk_len", C.c_uint32),
                ("bv", C.c_void_p), ("bv_len", C.c_uint32)]


class OracleModel:
    """Oracle forward_into (model.rs:7177-7358) over a model dict produced by
    rustyllm_amd.synth (the same bytes the HIP decoder consumes)."""

    def __init__(self, model, storage_len: int, threads: int = 0, kv_bf16: bool = False):
        cfg = model["config"]
        self.model = model
        self.cfg = cfg
        self.vocab = cfg["vocab"]
        self.kv_bf16 = kv_bf16
        c = OrcConfig(cfg["n_layers"], cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"],
                      cfg["value_dim"], cfg["hidden_dim"], cfg["vocab"], storage_len, cfg.get("sliding_window", 0),
                      1 if cfg.get("neox") else 0, cfg["eps"], 1 if kv_bf16 else 0)
        if threads:
            lib.orc_set_threads(threads)
        self.h = lib.orc_model_create(C.byref(c))
        self._keep = []
        for l, layer in enumerate(model["layers"]):
            L = OrcLayer()
            for i, (arr, dt, rows) in enumerate(layer["w"]):
                L.w[i] = ptr(arr)
                L.w_len[i] = arr.nbytes
                L.w_rows[i] = rows
                L.w_type[i] = dt
            L.attn_norm = ptr(layer["attn_norm"])
            L.ffn_norm = ptr(layer["ffn_norm"])
            for nm in ("bq", "bk", "bv"):
                b = layer.get(nm)
                if b is not None:
                    setattr(L, nm, ptr(b))
                    setattr(L, nm + "_len", b.size)
            lib.orc_model_set_layer(self.h, l, C.byref(L))
        out_w, out_dt = model["output"]
        emb_w, emb_dt = model["token_embd"]
        lib.orc_model_set_output(self.h, ptr(model["output_norm"]), ptr(out_w), out_dt, ptr(emb_w), emb_dt,
                                 ptr(model["inv_freq"]))

    def forward(self, token: int, pos: int, want_logits: bool = True, start_t: int = -1):
        """start_t >= 0: every layer attends start_t..pos (the resident
        decoder's start_t); -1: the model's own range."""
        logits = np.zeros(self.vocab, np.float32)
        lib.orc_model_forward_from(self.h, token, pos, start_t, ptr(logits), 1 if want_logits else 0)
        return logits

    def kv(self, layer: int, storage_len: int):
        cfg = self.cfg
        kd = cfg["n_kv_heads"] * cfg["head_dim"]
        vd = cfg["n_kv_heads"] * cfg["value_dim"]
        kp = lib.orc_model_kv(self.h, layer, 0)
        vp = lib.orc_model_kv(self.h, layer, 1)
        if self.kv_bf16:  # uint16 bf16 elements
            u16 = C.POINTER(C.c_uint16)
            k = np.ctypeslib.as_array(C.cast(kp, u16), shape=(storage_len * kd,))
            v = np.ctypeslib.as_array(C.cast(vp, u16), shape=(storage_len * vd,))
            return k, v
        k = np.ctypeslib.as_array(kp, shape=(storage_len * kd,))
        v = np.ctypeslib.as_array(vp, shape=(storage_len * vd,))
        return k, v

    def generate(self, prompt, n_gen, penalty=1.1, start_pos=0):
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(max(n_gen, 1), np.uint32)
        logits = np.zeros(self.vocab, np.float32)
        n = lib.orc_model_generate(self.h, ptr(p), p.size, start_pos, n_gen, penalty, ptr(out), ptr(logits))
        return out[:n], logits

    def __del__(self):
        try:
            lib.orc_model_free(self.h)
        except Exception:
            pass
