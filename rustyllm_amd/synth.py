"""Seeded synthetic models of the benchmark shapes.

A model is a dict of numpy arrays laid out exactly as the GGUF tensors are
(raw block bytes for quantized weights, f32 for norms and biases), so the same
bytes feed the HIP decoder, the CPU checker and the GGUF writer:

    {"config": {...},
     "token_embd": (bytes, ggml_type), "output": (bytes, ggml_type),
     "output_norm": f32[dim], "inv_freq": f32[head_dim/2],
     "layers": [{"w": [(bytes, ggml_type, rows) x 7], "attn_norm", "ffn_norm",
                 "bq"/"bk"/"bv" (optional)}]}

Weight order is wq, wk, wv, wo, gate, up, down (the reference's
ResidentLayerDesc order, src/metal.rs:344-360).  Weights are N(0, 0.02), norms
1.0, biases N(0, 0.02); each tensor has its own seed derived from the model
seed, and rows are generated independently, so the bytes do not depend on the
thread count.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import build as _build

F32, Q8_0, Q4_K, Q6_K, MXFP4 = 0, 8, 12, 14, 39
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), MXFP4: (32, 17)}

# Shapes from BASELINE.json configs.
CONFIGS = {
    # small shape used by the parity tests (tiny_standard_model-like: 2 layers, dim 256)
    "tiny-q4km": dict(arch="llama", n_layers=2, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, hidden_dim=512,
                      vocab=1024, theta=10000.0, eps=1e-5, quant="q4k_m"),
    "tiny-q8": dict(arch="llama", n_layers=2, dim=256, n_heads=4, n_kv_heads=1, head_dim=64, hidden_dim=512,
                    vocab=1024, theta=10000.0, eps=1e-5, quant="q8_0"),
    # ffn_down rows of 32 blocks (the row-split K-quant tiles) at a test's size
    "tiny-q4km-wide": dict(arch="llama", n_layers=2, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, hidden_dim=8192,
                           vocab=1024, theta=10000.0, eps=1e-5, quant="q4k_m"),
    "tiny-qwen": dict(arch="qwen2", n_layers=2, dim=512, n_heads=4, n_kv_heads=1, head_dim=128, hidden_dim=768,
                      vocab=1024, theta=1000000.0, eps=1e-6, quant="q4k_m", qkv_bias=True),
    # config 1: TinyLlama-1.1B shape, all Q8_0
    "tinyllama-1.1b-q8_0": dict(arch="llama", n_layers=22, dim=2048, n_heads=32, n_kv_heads=4, head_dim=64,
                                hidden_dim=5632, vocab=32000, theta=10000.0, eps=1e-5, quant="q8_0"),
    # config 3: Llama-3-8B shape, Q4_K_M mix
    "llama3-8b-q4km": dict(arch="llama", n_layers=32, dim=4096, n_heads=32, n_kv_heads=8, head_dim=128,
                           hidden_dim=14336, vocab=128256, theta=500000.0, eps=1e-5, quant="q4k_m"),
    # config 4: Qwen2.5-14B shape (qwen2 arch: NeoX RoPE, QKV bias)
    "qwen2.5-14b-q4km": dict(arch="qwen2", n_layers=48, dim=5120, n_heads=40, n_kv_heads=8, head_dim=128,
                             hidden_dim=13824, vocab=152064, theta=1000000.0, eps=1e-6, quant="q4k_m",
                             qkv_bias=True),
}


def _load():
    if not os.path.exists(_build.SYNTH_LIB):
        _build.build_synth()
    lib = C.CDLL(_build.SYNTH_LIB)
    lib.synth_row_bytes.restype = C.c_int64
    lib.synth_row_bytes.argtypes = [C.c_int, C.c_int64]
    lib.synth_normal_f32.restype = None
    lib.synth_normal_f32.argtypes = [C.c_uint64, C.c_int64, C.c_int64, C.c_float, C.c_float, C.c_void_p]
    lib.synth_quantize.restype = C.c_int
    lib.synth_quantize.argtypes = [C.c_int, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p]
    lib.synth_normal_quantized.restype = C.c_int
    lib.synth_normal_quantized.argtypes = [C.c_int, C.c_uint64, C.c_int64, C.c_int64, C.c_float, C.c_void_p]
    lib.synth_token_ids.restype = None
    lib.synth_token_ids.argtypes = [C.c_uint64, C.c_int64, C.c_uint32, C.c_void_p]
    lib.synth_rope_inv_freq.restype = None
    lib.synth_rope_inv_freq.argtypes = [C.c_float, C.c_int64, C.c_float, C.c_void_p]
    lib.synth_rope_inv_freq_gpt_oss.restype = None
    lib.synth_rope_inv_freq_gpt_oss.argtypes = [C.c_float, C.c_int64, C.c_float, C.c_int64, C.c_void_p, C.c_void_p]
    return lib


lib = _load()


def row_bytes(ggml_type: int, cols: int) -> int:
    return int(lib.synth_row_bytes(ggml_type, cols))


def normal_f32(seed: int, rows: int, cols: int, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    lib.synth_normal_f32(seed, rows, cols, std, mean, out.ctypes.data)
    return out


def quantize(ggml_type: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    out = np.empty(rows * row_bytes(ggml_type, cols), np.uint8)
    if lib.synth_quantize(ggml_type, x.ctypes.data, rows, cols, out.ctypes.data) != 1:
        raise ValueError(f"cannot quantize to type {ggml_type} with cols={cols}")
    return out


def normal_quantized(ggml_type: int, seed: int, rows: int, cols: int, std: float = 0.02) -> np.ndarray:
    out = np.empty(rows * row_bytes(ggml_type, cols), np.uint8)
    if lib.synth_normal_quantized(ggml_type, seed, rows, cols, std, out.ctypes.data) != 1:
        raise ValueError(f"cannot quantize to type {ggml_type} with cols={cols}")
    return out


def token_ids(seed: int, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib.synth_token_ids(seed, n, vocab, out.ctypes.data)
    return out


def rope_inv_freq(theta: float, head_dim: int, scaling: float = 1.0) -> np.ndarray:
    out = np.empty(head_dim // 2, np.float32)
    lib.synth_rope_inv_freq(theta, head_dim, scaling, out.ctypes.data)
    return out


def layer_types(quant: str, layer: int):
    """GGML types of (wq, wk, wv, wo, gate, up, down) for a quant mix."""
    if quant == "q8_0":
        return [Q8_0] * 7
    if quant == "q4k_m":
        # Q4_K_M as BASELINE.json describes it: Q4_K for attn_q/k/o and
        # ffn_gate/up, Q6_K for attn_v and for ffn_down on half of the layers.
        down = Q6_K if layer % 2 == 0 else Q4_K
        return [Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q4_K, down]
    if quant == "q4_k":
        return [Q4_K] * 7
    if quant == "q6_k":
        return [Q6_K] * 7
    raise ValueError(quant)


def make_model(name_or_cfg, seed: int = 1234) -> dict:
    cfg = dict(CONFIGS[name_or_cfg]) if isinstance(name_or_cfg, str) else dict(name_or_cfg)
    cfg.setdefault("value_dim", cfg["head_dim"])
    cfg.setdefault("neox", cfg.get("arch") in ("qwen2", "qwen3"))
    dim, hd, vd = cfg["dim"], cfg["head_dim"], cfg["value_dim"]
    nh, nkv, hid, vocab = cfg["n_heads"], cfg["n_kv_heads"], cfg["hidden_dim"], cfg["vocab"]
    quant = cfg["quant"]
    tensor_seed = [seed * 1000003]

    def next_seed():
        tensor_seed[0] += 7919
        return tensor_seed[0]

    layers = []
    for l in range(cfg["n_layers"]):
        types = layer_types(quant, l)
        shapes = [(nh * hd, dim), (nkv * hd, dim), (nkv * vd, dim), (dim, nh * vd), (hid, dim), (hid, dim),
                  (dim, hid)]
        w = []
        for t, (rows, cols) in zip(types, shapes):
            w.append((normal_quantized(t, next_seed(), rows, cols, 0.02), t, rows))
        layer = {"w": w, "attn_norm": np.ones(dim, np.float32), "ffn_norm": np.ones(dim, np.float32)}
        if cfg.get("qkv_bias"):
            layer["bq"] = normal_f32(next_seed(), 1, nh * hd, 0.02).reshape(-1)
            layer["bk"] = normal_f32(next_seed(), 1, nkv * hd, 0.02).reshape(-1)
            layer["bv"] = normal_f32(next_seed(), 1, nkv * vd, 0.02).reshape(-1)
        layers.append(layer)
    if quant == "q8_0":
        emb_t, out_t = Q8_0, Q8_0
    else:
        emb_t, out_t = Q4_K, Q6_K
    model = {
        "config": cfg,
        "layers": layers,
        "token_embd": (normal_quantized(emb_t, next_seed(), vocab, dim, 0.02), emb_t),
        "output": (normal_quantized(out_t, next_seed(), vocab, dim, 0.02), out_t),
        "output_norm": np.ones(dim, np.float32),
        "inv_freq": rope_inv_freq(cfg["theta"], hd, 1.0),
    }
    return model


# gpt-oss family: Q8_0 attention, router and output,
# MXFP4 experts, learned sinks, sliding window on even layers, YaRN RoPE.
GPTOSS_CONFIGS = {
    # parity shape: f32-activation paths (dim % 256 != 0), a Q8_K wo (n_heads*head_dim = 256)
    "tiny-gptoss": dict(n_layers=3, dim=160, n_heads=4, n_kv_heads=2, head_dim=64, hidden_dim=96, n_experts=6,
                        top_k=2, vocab=500, window=8, theta=150000.0, rope_scaling=32.0, rope_orig_ctx=4096,
                        eps=1e-5),
    # the same with the real 128-position window: the ring then has enough
    # slots for the main (LDS-tiled) attention kernels
    "tiny-gptoss-w128": dict(n_layers=3, dim=160, n_heads=4, n_kv_heads=2, head_dim=64, hidden_dim=96, n_experts=6,
                             top_k=2, vocab=500, window=128, theta=150000.0, rope_scaling=32.0, rope_orig_ctx=4096,
                             eps=1e-5),
    "gpt-oss-20b": dict(n_layers=24, dim=2880, n_heads=64, n_kv_heads=8, head_dim=64, hidden_dim=2880,
                        n_experts=32, top_k=4, vocab=201088, window=128, theta=150000.0, rope_scaling=32.0,
                        rope_orig_ctx=4096, eps=1e-5),
}


def rope_gpt_oss(theta: float, head_dim: int, scaling: float, orig_ctx: int):
    """build_rope_inv_freq_gpt_oss (src/model.rs:3059-3098): YaRN frequencies
    and the concentration 0.1 ln(scaling) + 1, in f32 with libm logf/powf
    (csrc/synth.cpp)."""
    inv = np.empty(head_dim // 2, np.float32)
    conc = C.c_float(0.0)
    lib.synth_rope_inv_freq_gpt_oss(theta, head_dim, scaling, orig_ctx, inv.ctypes.data, C.addressof(conc))
    return inv, float(conc.value)


def make_gptoss(name_or_cfg, seed: int = 1234) -> dict:
    """A gpt-oss model: per layer wq/wk/wv/wo (Q8_0) with biases, sinks,
    attn/post-attention norms, router (Q8_0) + bias, expert-major MXFP4
    gate/up/down with f32 biases; Q8_0 embedding and output."""
    cfg = dict(GPTOSS_CONFIGS[name_or_cfg]) if isinstance(name_or_cfg, str) else dict(name_or_cfg)
    cfg.setdefault("value_dim", cfg["head_dim"])
    cfg["arch"] = "gpt-oss"
    dim, hd, vd = cfg["dim"], cfg["head_dim"], cfg["value_dim"]
    nh, nkv, hid, ne, vocab = cfg["n_heads"], cfg["n_kv_heads"], cfg["hidden_dim"], cfg["n_experts"], cfg["vocab"]
    seed_box = [seed * 1000003 + 17]

    def ns():
        seed_box[0] += 7919
        return seed_box[0]

    def vec(n, std):
        return normal_f32(ns(), 1, n, std).reshape(-1)

    layers = []
    for _ in range(cfg["n_layers"]):
        L = {
            "wq": (normal_quantized(Q8_0, ns(), nh * hd, dim, 0.02), Q8_0),
            "wk": (normal_quantized(Q8_0, ns(), nkv * hd, dim, 0.02), Q8_0),
            "wv": (normal_quantized(Q8_0, ns(), nkv * vd, dim, 0.02), Q8_0),
            "wo": (normal_quantized(Q8_0, ns(), dim, nh * vd, 0.02), Q8_0),
            "bq": vec(nh * hd, 0.02), "bk": vec(nkv * hd, 0.02), "bv": vec(nkv * vd, 0.02), "bo": vec(dim, 0.02),
            "sinks": vec(nh, 1.0),
            "attn_norm": np.ones(dim, np.float32), "post_attn_norm": np.ones(dim, np.float32),
            "router": normal_quantized(Q8_0, ns(), ne, dim, 0.02), "router_bias": vec(ne, 0.02),
            "gate_exps": normal_quantized(MXFP4, ns(), ne * hid, dim, 0.02),
            "up_exps": normal_quantized(MXFP4, ns(), ne * hid, dim, 0.02),
            "down_exps": normal_quantized(MXFP4, ns(), ne * dim, hid, 0.02),
            "gate_exps_bias": normal_f32(ns(), ne, hid, 0.02), "up_exps_bias": normal_f32(ns(), ne, hid, 0.02),
            "down_exps_bias": normal_f32(ns(), ne, dim, 0.02),
        }
        layers.append(L)
    inv, conc = rope_gpt_oss(cfg["theta"], hd, cfg["rope_scaling"], cfg["rope_orig_ctx"])
    return {
        "config": cfg,
        "layers": layers,
        "token_embd": (normal_quantized(Q8_0, ns(), vocab, dim, 0.02), Q8_0),
        "output": (normal_quantized(Q8_0, ns(), vocab, dim, 0.02), Q8_0),
        "output_norm": np.ones(dim, np.float32),
        "inv_freq": inv,
        "concentration": conc,
    }


def weight_bytes(model: dict, include_embedding: bool = False) -> int:
    """Bytes of every weight read per decode token (the embedding row is one row)."""
    total = 0
    for layer in model["layers"]:
        for arr, _, _ in layer["w"]:
            total += arr.nbytes
        total += layer["attn_norm"].nbytes + layer["ffn_norm"].nbytes
        for nm in ("bq", "bk", "bv"):
            if layer.get(nm) is not None:
                total += layer[nm].nbytes
    total += model["output"][0].nbytes + model["output_norm"].nbytes
    if include_embedding:
        total += model["token_embd"][0].nbytes
    return total
