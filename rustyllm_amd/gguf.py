"""GGUF v3 files for the decode path: a reader that follows the reference's
parser (src/gguf.rs) and model loaders (Config::from_gguf, src/model.rs:
40-120; load_model :3573-3724 and its attn_qkv split :3731-3860;
load_gpt_oss_model :5180-5420), and a writer for the synthetic models of
rustyllm_amd.synth, so that BASELINE's "GGUF written from a seed" exists as a
file.

The file layout (little-endian): "GGUF", u32 version, u64 tensor count, u64
metadata count; metadata entries (GGUF string key, u32 value type, value);
tensor infos (string name, u32 n_dims, u64 dims (fastest first), u32 GGML
type, u64 offset from the data start); tensor data from the first multiple of
general.alignment (default 32) after the header.  Value types 0-12 are
u8, i8, u16, i16, u32, i32, f32, bool, string, array (u32 element type, u64
count, elements), u64, i64, f64 (src/gguf.rs:301-330).

The device-side loader (rusty_hip_resident_load_gguf) parses the same files
natively; load_model here returns the same model dict as synth.make_model /
synth.make_gptoss, which the oracle and the ctypes decoders consume.
"""
from __future__ import annotations

import mmap
import os
import struct

import numpy as np

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, BF16, MXFP4 = 0, 1, 2, 8, 12, 14, 30, 39
# (elements, bytes) per block, GGMLType::block_size / block_bytes (src/gguf.rs:59-87)
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
         Q8_0: (32, 34), 9: (32, 36), Q4_K: (256, 144), 13: (256, 176), Q6_K: (256, 210), MXFP4: (32, 17)}

# metadata value types (src/gguf.rs:301-330)
U8, I8, U16, I16, U32, I32, FLOAT32, BOOL, STRING, ARRAY, U64, I64, FLOAT64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", FLOAT32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", FLOAT64: "<d"}


def data_size(dtype: int, n: int) -> int | None:
    """GGMLType::data_size (src/gguf.rs:89-107): whole blocks for n elements."""
    if dtype not in BLOCK:
        return None
    be, bb = BLOCK[dtype]
    return -(-n // be) * bb


class TensorInfo:
    def __init__(self, name: str, dims, dtype: int, offset: int):
        self.name, self.dims, self.dtype, self.offset = name, list(dims), dtype, offset

    def numel(self) -> int:
        n = 1
        for d in self.dims:
            n *= int(d)
        return n


class Meta:
    """A typed metadata value (type id + python value; arrays hold Meta items)."""

    def __init__(self, vtype: int, value):
        self.vtype, self.value = vtype, value

    def as_u32(self):
        """MetaValue::as_u32 (src/gguf.rs:131-141): integer types wrap to u32."""
        if self.vtype in (U32, I32, U64, I64, U8, U16):
            return int(self.value) & 0xFFFFFFFF
        return None

    def as_f32(self):
        if self.vtype in (FLOAT32, FLOAT64):
            return float(np.float32(self.value))
        return None

    def as_str(self):
        return self.value if self.vtype == STRING else None

    def as_u32_array(self):
        if self.vtype != ARRAY:
            return None
        return [int(v.value) for v in self.value if v.vtype in (U8, U16, U32, U64, I8, I16, I32, I64)
                and 0 <= int(v.value) <= 0xFFFFFFFF]


class _Cursor:
    def __init__(self, buf):
        self.b, self.pos = buf, 0

    def take(self, fmt):
        v = struct.unpack_from(fmt, self.b, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def string(self) -> str:
        n = self.take("<Q")
        s = bytes(self.b[self.pos:self.pos + n]).decode("utf-8", errors="replace")
        self.pos += n
        return s

    def value(self, vtype: int) -> Meta:
        if vtype in _SCALAR:
            v = self.take(_SCALAR[vtype])
            return Meta(vtype, bool(v) if vtype == BOOL else v)
        if vtype == STRING:
            return Meta(STRING, self.string())
        if vtype == ARRAY:
            et = self.take("<I")
            n = self.take("<Q")
            return Meta(ARRAY, [self.value(et) for _ in range(n)])
        raise ValueError(f"Unknown GGUF metadata value type {vtype}")


class GGUFFile:
    """GGUFFile::parse (src/gguf.rs:338-418) over a read-only mapping."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        size = os.fstat(self._f.fileno()).st_size
        if size < 4:
            raise ValueError("File too small for GGUF header")
        self.buf = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        if self.buf[:4] != b"GGUF":
            raise ValueError("Invalid GGUF magic: 0x%08X" % struct.unpack_from("<I", self.buf, 0)[0])
        c = _Cursor(self.buf)
        c.pos = 4
        self.version = c.take("<I")
        n_tensors = c.take("<Q")
        n_kv = c.take("<Q")
        self.metadata = {}
        for _ in range(n_kv):
            key = c.string()
            self.metadata[key] = c.value(c.take("<I"))
        self.tensors = []
        for _ in range(n_tensors):
            name = c.string()
            nd = c.take("<I")
            dims = [c.take("<Q") for _ in range(nd)]
            dt = c.take("<I")
            off = c.take("<Q")
            self.tensors.append(TensorInfo(name, dims, dt, off))
        align = self.get_u32("general.alignment", 32)
        self.data_offset = -(-c.pos // align) * align
        self.index = {t.name: t for t in self.tensors}

    def close(self):
        """Unmaps the file once no tensor view refers to it any more (views
        handed out by tensor_bytes keep the mapping alive until dropped)."""
        try:
            self.buf.close()
        except BufferError:
            return
        self._f.close()

    def get_u32(self, key: str, default: int) -> int:
        v = self.metadata.get(key)
        r = v.as_u32() if v is not None else None
        return default if r is None else r

    def get_f32(self, key: str, default: float) -> float:
        v = self.metadata.get(key)
        r = v.as_f32() if v is not None else None
        return float(np.float32(default)) if r is None else r

    def get_str(self, key: str):
        v = self.metadata.get(key)
        return v.as_str() if v is not None else None

    def tensor_bytes(self, name: str) -> np.ndarray:
        """The tensor's raw bytes, a view of the mapping (data_size of its
        element count, as load_weight reads them)."""
        t = self.index[name]
        n = data_size(t.dtype, t.numel())
        if n is None:
            raise ValueError(f"Unsupported tensor type/size for {name}: {t.dtype}")
        start = self.data_offset + t.offset
        if start + n > len(self.buf):
            raise ValueError(f"Tensor {name}: offset {start} + byte_size {n} exceeds mmap length {len(self.buf)}")
        return np.frombuffer(self.buf, np.uint8, n, start)

    def f32(self, name: str) -> np.ndarray:
        t = self.index[name]
        b = self.tensor_bytes(name)
        if t.dtype == F32:
            return b.view(np.float32).copy()
        if t.dtype == F16:
            return b.view(np.float16).astype(np.float32)
        if t.dtype == BF16:
            return (b.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        raise ValueError(f"{name}: not a float tensor ({t.dtype})")


def config_from_gguf(g: GGUFFile) -> dict:
    """Config::from_gguf (src/model.rs:40-120)."""
    arch = g.get_str("general.architecture") or "llama"
    p = arch
    dim = g.get_u32(f"{p}.embedding_length", 0)
    hc = g.metadata.get(f"{p}.attention.head_count")
    n_heads = g.get_u32(f"{p}.attention.head_count", 0)
    if hc is not None and hc.vtype == ARRAY:
        n_heads = max(n_heads, max(hc.as_u32_array() or [0]))
    n_kv = g.get_u32(f"{p}.attention.head_count_kv", n_heads)
    rope_dim = g.get_u32(f"{p}.rope.dimension_count", 0)
    default_hd = dim // n_heads if dim > 0 and n_heads > 0 else rope_dim
    head_dim = g.get_u32(f"{p}.attention.key_length", default_hd)
    value_dim = g.get_u32(f"{p}.attention.value_length", head_dim)
    tok = g.metadata.get("tokenizer.ggml.tokens")
    # as_string_array (src/gguf.rs:161-176): only the string entries count
    n_tok = sum(1 for v in tok.value if v.vtype == STRING) if tok is not None and tok.vtype == ARRAY else 0
    vocab = max(g.get_u32(f"{p}.vocab_size", 0), n_tok)
    ff = g.metadata.get(f"{p}.feed_forward_length")
    hidden = 0
    if ff is not None:
        hidden = ff.as_u32()
        if hidden is None and ff.vtype == ARRAY:
            hidden = max([v.as_u32() for v in ff.value if v.as_u32() is not None] or [0])
        hidden = hidden or 0
    return dict(arch=arch, dim=dim, hidden_dim=hidden, n_layers=g.get_u32(f"{p}.block_count", 0), n_heads=n_heads,
                n_kv_heads=n_kv, vocab=vocab, max_seq_len=g.get_u32(f"{p}.context_length", 2048),
                theta=g.get_f32(f"{p}.rope.freq_base", 10000.0),
                eps=g.get_f32(f"{p}.attention.layer_norm_rms_epsilon", 1e-5), head_dim=head_dim,
                value_dim=value_dim, window=g.get_u32(f"{p}.attention.sliding_window", 0),
                n_experts=g.get_u32(f"{p}.expert_count", 0), top_k=g.get_u32(f"{p}.expert_used_count", 0),
                rope_scaling=g.get_f32(f"{p}.rope.scaling.factor", 1.0),
                rope_orig_ctx=g.get_u32(f"{p}.rope.scaling.original_context_length", 0))


def _matrix(g: GGUFFile, name: str):
    t = g.index[name]
    rows = 1
    for d in t.dims[1:]:
        rows *= int(d)
    return g.tensor_bytes(name), t.dtype, rows, int(t.dims[0])


def load_model(path: str) -> dict:
    """The model dict synth.make_model / make_gptoss would give for this file:
    load_model (src/model.rs:3573-3724) for llama / qwen2, with the tied
    output fallback (:3653-3667), the head/value dim override from the
    attn_q / attn_v shapes (:3668-3724) and the fused attn_qkv split
    (:3731-3860); load_gpt_oss_model (:5180-5420) for gpt-oss.  Weight arrays
    are views of the file mapping."""
    g = GGUFFile(path)
    cfg = config_from_gguf(g)
    if cfg["arch"] == "gpt-oss":
        return _load_gptoss(g, cfg)
    L = cfg["n_layers"]
    # head_dim / value_dim from tensor shapes when they disagree with metadata
    for l in range(L):
        q = g.index.get(f"blk.{l}.attn_q.weight")
        v = g.index.get(f"blk.{l}.attn_v.weight")
        hd = vd = None
        if q is not None and len(q.dims) >= 2 and q.dims[0] == cfg["dim"] and q.dims[1] % cfg["n_heads"] == 0:
            hd = q.dims[1] // cfg["n_heads"]
        if v is not None and len(v.dims) >= 2 and v.dims[0] == cfg["dim"] and v.dims[1] % cfg["n_kv_heads"] == 0:
            vd = v.dims[1] // cfg["n_kv_heads"]
        if hd is not None:
            cfg["head_dim"] = int(hd)
        if vd is not None:
            cfg["value_dim"] = int(vd)
        if hd is not None and vd is not None:
            break
    nh, nkv, hd, vd, dim = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["value_dim"], cfg["dim"]
    q_rows, k_rows, v_rows = nh * hd, nkv * hd, nkv * vd
    cfg["neox"] = cfg["arch"] in ("qwen2", "qwen3")
    layers = []
    for l in range(L):
        lay = {}
        if f"blk.{l}.attn_q.weight" in g.index:
            mats = [_matrix(g, f"blk.{l}.attn_{n}.weight") for n in ("q", "k", "v")]
            for nm, n in (("bq", "q"), ("bk", "k"), ("bv", "v")):
                if f"blk.{l}.attn_{n}.bias" in g.index:
                    lay[nm] = g.f32(f"blk.{l}.attn_{n}.bias")
        else:
            qkv, t, rows, cols = _matrix(g, f"blk.{l}.attn_qkv.weight")
            rb = data_size(t, cols)
            mats = [(qkv[r0 * rb:(r0 + n) * rb], t, n, cols)
                    for r0, n in ((0, q_rows), (q_rows, k_rows), (q_rows + k_rows, v_rows))]
            if f"blk.{l}.attn_qkv.bias" in g.index:
                b = g.f32(f"blk.{l}.attn_qkv.bias")
                lay["bq"], lay["bk"], lay["bv"] = b[:q_rows], b[q_rows:q_rows + k_rows], b[q_rows + k_rows:]
        mats += [_matrix(g, f"blk.{l}.{n}.weight") for n in ("attn_output", "ffn_gate", "ffn_up", "ffn_down")]
        lay["w"] = [(m[0], m[1], m[2]) for m in mats]
        lay["attn_norm"] = g.f32(f"blk.{l}.attn_norm.weight")
        lay["ffn_norm"] = g.f32(f"blk.{l}.ffn_norm.weight")
        layers.append(lay)
    if "qkv_bias" not in cfg:
        cfg["qkv_bias"] = "bq" in layers[0]
    emb = _matrix(g, "token_embd.weight")
    out = _matrix(g, "output.weight") if "output.weight" in g.index else emb
    cfg["tied_output"] = "output.weight" not in g.index
    from . import synth
    return {"config": cfg, "layers": layers, "token_embd": (emb[0], emb[1]), "output": (out[0], out[1]),
            "output_norm": g.f32("output_norm.weight"),
            "inv_freq": synth.rope_inv_freq(cfg["theta"], cfg["head_dim"], 1.0), "_gguf": g}


def _load_gptoss(g: GGUFFile, cfg: dict) -> dict:
    from . import synth
    layers = []
    for l in range(cfg["n_layers"]):
        b = f"blk.{l}."
        lay = {nm: (_matrix(g, b + key)[0], g.index[b + key].dtype) for nm, key in
               (("wq", "attn_q.weight"), ("wk", "attn_k.weight"), ("wv", "attn_v.weight"),
                ("wo", "attn_output.weight"))}
        for nm, key in (("bq", "attn_q.bias"), ("bk", "attn_k.bias"), ("bv", "attn_v.bias"),
                        ("bo", "attn_output.bias"), ("sinks", "attn_sinks.weight"), ("attn_norm", "attn_norm.weight"),
                        ("post_attn_norm", "post_attention_norm.weight"), ("router_bias", "ffn_gate_inp.bias")):
            lay[nm] = g.f32(b + key)
        lay["router"] = g.tensor_bytes(b + "ffn_gate_inp.weight")
        for nm in ("gate_exps", "up_exps", "down_exps"):
            lay[nm] = g.tensor_bytes(b + f"ffn_{nm}.weight")
            bias = g.f32(b + f"ffn_{nm}.bias")
            t = g.index[b + f"ffn_{nm}.bias"]
            lay[nm + "_bias"] = bias.reshape(int(t.dims[1]), int(t.dims[0]))
        layers.append(lay)
    inv, conc = synth.rope_gpt_oss(cfg["theta"], cfg["head_dim"], cfg["rope_scaling"], cfg["rope_orig_ctx"])
    return {"config": cfg, "layers": layers,
            "token_embd": (g.tensor_bytes("token_embd.weight"), g.index["token_embd.weight"].dtype),
            "output": (g.tensor_bytes("output.weight"), g.index["output.weight"].dtype),
            "output_norm": g.f32("output_norm.weight"), "inv_freq": inv, "concentration": conc,
            "router_type": g.index["blk.0.ffn_gate_inp.weight"].dtype,
            "experts_type": g.index["blk.0.ffn_gate_exps.weight"].dtype, "_gguf": g}


# ---- writer --------------------------------------------------------------------------
def _enc_string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _enc_value(vtype: int, value) -> bytes:
    if vtype in _SCALAR:
        return struct.pack(_SCALAR[vtype], int(value) if vtype == BOOL else value)
    if vtype == STRING:
        return _enc_string(value)
    if vtype == ARRAY:
        et, items = value
        return struct.pack("<IQ", et, len(items)) + b"".join(_enc_value(et, v) for v in items)
    raise ValueError(vtype)


def write(path: str, metadata, tensors, alignment: int = 32, version: int = 3) -> None:
    """metadata: [(key, vtype, value)] (arrays: (elem_type, [values]));
    tensors: [(name, dims fastest-first, ggml type, bytes-like)].  Each
    tensor's data starts on an `alignment` boundary of the data section."""
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in metadata):
        metadata = list(metadata) + [("general.alignment", U32, alignment)]
    head = [b"GGUF", struct.pack("<IQQ", version, len(tensors), len(metadata))]
    for k, vt, v in metadata:
        head += [_enc_string(k), struct.pack("<I", vt), _enc_value(vt, v)]
    off = 0
    offsets = []
    for name, dims, dt, data in tensors:
        n = memoryview(data).nbytes
        need = data_size(dt, int(np.prod(dims)))
        if need is not None and n != need:
            raise ValueError(f"{name}: {n} bytes for dims {dims} of type {dt} (expected {need})")
        offsets.append(off)
        head += [_enc_string(name), struct.pack("<I", len(dims)), struct.pack(f"<{len(dims)}Q", *dims),
                 struct.pack("<IQ", dt, off)]
        off = -(-(off + n) // alignment) * alignment
    h = b"".join(head)
    pad = -(-len(h) // alignment) * alignment - len(h)
    with open(path, "wb") as f:
        f.write(h + b"\0" * pad)
        pos = 0
        for (name, dims, dt, data), o in zip(tensors, offsets):
            f.write(b"\0" * (o - pos))
            mv = memoryview(data).cast("B")
            f.write(mv)
            pos = o + mv.nbytes
        f.write(b"\0" * (-(-pos // alignment) * alignment - pos))


def _f32_bytes(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32)


def write_model(path: str, model: dict, tie_output: bool = False, fuse_qkv: bool = False) -> None:
    """Writes a rustyllm_amd.synth model with the metadata keys and tensor
    names the reference's loaders read.  tie_output leaves output.weight out
    (the loader then uses token_embd, src/model.rs:3653-3667); fuse_qkv
    stores blk.N.attn_qkv.weight (and .bias) instead of q/k/v
    (:3795-3859)."""
    c = model["config"]
    arch = c.get("arch", "llama")
    p = arch
    md = [("general.architecture", STRING, arch), ("general.name", STRING, f"synthetic {arch}"),
          (f"{p}.embedding_length", U32, c["dim"]), (f"{p}.block_count", U32, c["n_layers"]),
          (f"{p}.attention.head_count", U32, c["n_heads"]), (f"{p}.attention.head_count_kv", U32, c["n_kv_heads"]),
          (f"{p}.attention.key_length", U32, c["head_dim"]),
          (f"{p}.attention.value_length", U32, c.get("value_dim", c["head_dim"])),
          (f"{p}.feed_forward_length", U32, c["hidden_dim"]), (f"{p}.vocab_size", U32, c["vocab"]),
          (f"{p}.context_length", U32, c.get("max_seq_len", 4096)),
          (f"{p}.rope.freq_base", FLOAT32, float(c["theta"])),
          (f"{p}.attention.layer_norm_rms_epsilon", FLOAT32, float(c["eps"])),
          ("general.alignment", U32, 32)]
    if arch == "gpt-oss":
        md += [(f"{p}.attention.sliding_window", U32, c["window"]), (f"{p}.expert_count", U32, c["n_experts"]),
               (f"{p}.expert_used_count", U32, c["top_k"]),
               (f"{p}.rope.scaling.factor", FLOAT32, float(c["rope_scaling"])),
               (f"{p}.rope.scaling.original_context_length", U32, c["rope_orig_ctx"])]
    dim, vocab = c["dim"], c["vocab"]
    T = []

    def mat(name, arr, dt, rows, cols):
        T.append((name, [cols, rows], dt, np.ascontiguousarray(arr, np.uint8)))

    emb, et = model["token_embd"]
    mat("token_embd.weight", emb, et, vocab, dim)
    T.append(("output_norm.weight", [dim], F32, _f32_bytes(model["output_norm"])))
    if not tie_output:
        ow, ot = model["output"]
        mat("output.weight", ow, ot, vocab, dim)
    if arch == "gpt-oss":
        nh, nkv, hd, vd, hid, ne = (c["n_heads"], c["n_kv_heads"], c["head_dim"], c.get("value_dim", c["head_dim"]),
                                    c["hidden_dim"], c["n_experts"])
        for l, L in enumerate(model["layers"]):
            b = f"blk.{l}."
            for nm, key, rows, cols in (("wq", "attn_q", nh * hd, dim), ("wk", "attn_k", nkv * hd, dim),
                                        ("wv", "attn_v", nkv * vd, dim), ("wo", "attn_output", dim, nh * vd)):
                mat(b + key + ".weight", L[nm][0], L[nm][1], rows, cols)
            for nm, key in (("bq", "attn_q.bias"), ("bk", "attn_k.bias"), ("bv", "attn_v.bias"),
                            ("bo", "attn_output.bias"), ("sinks", "attn_sinks.weight"),
                            ("attn_norm", "attn_norm.weight"), ("post_attn_norm", "post_attention_norm.weight"),
                            ("router_bias", "ffn_gate_inp.bias")):
                a = _f32_bytes(L[nm])
                T.append((b + key, [a.size], F32, a))
            mat(b + "ffn_gate_inp.weight", L["router"], model.get("router_type", Q8_0), ne, dim)
            et_ = model.get("experts_type", MXFP4)
            for nm, rows, cols in (("gate_exps", hid, dim), ("up_exps", hid, dim), ("down_exps", dim, hid)):
                T.append((b + f"ffn_{nm}.weight", [cols, rows, ne], et_, np.ascontiguousarray(L[nm], np.uint8)))
                bias = _f32_bytes(L[nm + "_bias"])
                T.append((b + f"ffn_{nm}.bias", [rows, ne], F32, bias))
    else:
        names = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")
        cols_of = [dim, dim, dim, c["n_heads"] * c.get("value_dim", c["head_dim"]), dim, dim, c["hidden_dim"]]
        for l, L in enumerate(model["layers"]):
            b = f"blk.{l}."
            w = L["w"]
            if fuse_qkv:
                if len({w[0][1], w[1][1], w[2][1]}) != 1:
                    raise ValueError("a fused attn_qkv tensor has one type")
                rows = w[0][2] + w[1][2] + w[2][2]
                data = np.concatenate([np.ascontiguousarray(w[i][0], np.uint8) for i in range(3)])
                T.append((b + "attn_qkv.weight", [dim, rows], w[0][1], data))
                if L.get("bq") is not None:
                    bb = _f32_bytes(np.concatenate([L["bq"], L["bk"], L["bv"]]))
                    T.append((b + "attn_qkv.bias", [bb.size], F32, bb))
                first = 3
            else:
                first = 0
                for nm, key in (("bq", "attn_q"), ("bk", "attn_k"), ("bv", "attn_v")):
                    if L.get(nm) is not None:
                        a = _f32_bytes(L[nm])
                        T.append((b + key + ".bias", [a.size], F32, a))
            for i in range(first, 7):
                arr, dt, rows = w[i]
                mat(b + names[i] + ".weight", arr, dt, rows, cols_of[i])
            T.append((b + "attn_norm.weight", [dim], F32, _f32_bytes(L["attn_norm"])))
            T.append((b + "ffn_norm.weight", [dim], F32, _f32_bytes(L["ffn_norm"])))
    write(path, md, T)
