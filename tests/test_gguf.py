"""GGUF v3 reader / writer (rustyllm_amd/gguf.py) against the format as the
reference parses it (src/gguf.rs) and the loaders' rules (Config::from_gguf,
src/model.rs:40-120; load_model :3573-3860; load_gpt_oss_model
:5180-5420).  CPU only."""
import struct

import numpy as np
import pytest

from rustyllm_amd import gguf, synth


def _same_model(a, b):
    ca, cb = a["config"], b["config"]
    for k in ("n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "value_dim", "hidden_dim", "vocab"):
        assert ca[k] == cb[k], k
    assert np.float32(ca["eps"]) == np.float32(cb["eps"]) and np.float32(ca["theta"]) == np.float32(cb["theta"])
    assert np.array_equal(np.asarray(a["token_embd"][0]), np.asarray(b["token_embd"][0]))
    assert a["token_embd"][1] == b["token_embd"][1]
    assert np.array_equal(np.asarray(a["output"][0]), np.asarray(b["output"][0]))
    assert np.array_equal(a["output_norm"], b["output_norm"])
    assert np.array_equal(a["inv_freq"].view(np.uint32), b["inv_freq"].view(np.uint32))


@pytest.mark.parametrize("name", ["tiny-q4km", "tiny-qwen", "tiny-q8"])
def test_standard_round_trip(tmp_path, name):
    m = synth.make_model(name, seed=3)
    p = str(tmp_path / f"{name}.gguf")
    gguf.write_model(p, m)
    r = gguf.load_model(p)
    _same_model(m, r)
    assert r["config"]["neox"] == m["config"]["neox"]
    for La, Lb in zip(m["layers"], r["layers"]):
        for (wa, ta, ra), (wb, tb, rb) in zip(La["w"], Lb["w"]):
            assert ta == tb and ra == rb and np.array_equal(wa, wb)
        for nm in ("attn_norm", "ffn_norm", "bq", "bk", "bv"):
            if La.get(nm) is not None:
                assert np.array_equal(La[nm], Lb[nm]), nm
            else:
                assert Lb.get(nm) is None
    g = r["_gguf"]
    assert g.version == 3 and g.data_offset % 32 == 0
    for t in g.tensors:
        assert t.offset % 32 == 0


def test_tied_output_and_fused_qkv(tmp_path):
    m = synth.make_model("tiny-q8", seed=4)
    p = str(tmp_path / "tied.gguf")
    gguf.write_model(p, m, tie_output=True, fuse_qkv=True)
    r = gguf.load_model(p)
    g = r["_gguf"]
    assert "output.weight" not in g.index and "blk.0.attn_qkv.weight" in g.index
    assert r["config"]["tied_output"]
    assert np.array_equal(np.asarray(r["output"][0]), np.asarray(m["token_embd"][0]))  # :3653-3667
    for La, Lb in zip(m["layers"], r["layers"]):
        for (wa, ta, ra), (wb, tb, rb) in zip(La["w"][:3], Lb["w"][:3]):
            assert ta == tb and ra == rb and np.array_equal(wa, wb)
    q = synth.make_model("tiny-qwen", seed=4)  # fused bias split too
    q["layers"] = [dict(L, w=[(a, synth.Q4_K if i < 3 else t, r) for i, (a, t, r) in enumerate(L["w"])])
                   for L in q["layers"]]
    for L in q["layers"]:  # make q/k/v one type for the fused tensor
        L["w"][2] = (synth.normal_quantized(synth.Q4_K, 9, L["w"][2][2], q["config"]["dim"]), synth.Q4_K,
                     L["w"][2][2])
    p2 = str(tmp_path / "qkv_bias.gguf")
    gguf.write_model(p2, q, fuse_qkv=True)
    r2 = gguf.load_model(p2)
    for La, Lb in zip(q["layers"], r2["layers"]):
        for nm in ("bq", "bk", "bv"):
            assert np.array_equal(La[nm], Lb[nm])
        assert np.array_equal(La["w"][2][0], Lb["w"][2][0])


def test_gptoss_round_trip(tmp_path):
    m = synth.make_gptoss("tiny-gptoss", seed=5)
    p = str(tmp_path / "gptoss.gguf")
    gguf.write_model(p, m)
    r = gguf.load_model(p)
    _same_model(m, r)
    c = r["config"]
    for k in ("window", "n_experts", "top_k", "rope_orig_ctx"):
        assert c[k] == m["config"][k], k
    assert np.float32(c["rope_scaling"]) == np.float32(m["config"]["rope_scaling"])
    assert r["concentration"] == m["concentration"]
    for La, Lb in zip(m["layers"], r["layers"]):
        for nm in ("wq", "wk", "wv", "wo"):
            assert La[nm][1] == Lb[nm][1] and np.array_equal(La[nm][0], Lb[nm][0])
        for nm in ("bq", "bk", "bv", "bo", "sinks", "attn_norm", "post_attn_norm", "router_bias", "router",
                   "gate_exps", "up_exps", "down_exps", "gate_exps_bias", "up_exps_bias", "down_exps_bias"):
            assert np.array_equal(np.asarray(La[nm]), np.asarray(Lb[nm])), nm
    g = r["_gguf"]
    t = g.index["blk.0.ffn_gate_exps.weight"]
    assert t.dims == [m["config"]["dim"], m["config"]["hidden_dim"], m["config"]["n_experts"]]  # [cols, rows, experts]


def _s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def test_parser_on_hand_built_bytes(tmp_path):
    """A file assembled byte by byte from the format (not by the writer):
    every scalar value type, a string array, a nested array, a custom
    alignment of 64, and a tensor whose data starts at the aligned offset."""
    md = [
        _s("a.u8") + struct.pack("<IB", 0, 200), _s("a.i8") + struct.pack("<Ib", 1, -5),
        _s("a.u16") + struct.pack("<IH", 2, 65000), _s("a.i16") + struct.pack("<Ih", 3, -30000),
        _s("a.u32") + struct.pack("<II", 4, 4000000000), _s("a.i32") + struct.pack("<Ii", 5, -7),
        _s("a.f32") + struct.pack("<If", 6, 1.5), _s("a.bool") + struct.pack("<IB", 7, 1),
        _s("a.str") + struct.pack("<I", 8) + _s("héllo"),
        _s("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, 3) + _s("x") + _s("yy") + _s("zzz"),
        _s("a.nested") + struct.pack("<IIQ", 9, 9, 2) + struct.pack("<IQ", 4, 2) + struct.pack("<II", 1, 2)
        + struct.pack("<IQ", 4, 1) + struct.pack("<I", 3),
        _s("a.u64") + struct.pack("<IQ", 10, 2 ** 40 + 3), _s("a.i64") + struct.pack("<Iq", 11, -2 ** 40),
        _s("a.f64") + struct.pack("<Id", 12, 0.1),
        _s("general.alignment") + struct.pack("<II", 4, 64),
        _s("general.architecture") + struct.pack("<I", 8) + _s("llama"),
    ]
    ti = _s("t.weight") + struct.pack("<I", 2) + struct.pack("<QQ", 32, 2) + struct.pack("<IQ", 8, 0)
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, len(md)) + b"".join(md) + ti
    data_off = -(-len(head) // 64) * 64
    payload = bytes(range(68))  # two Q8_0 blocks of 34 bytes
    p = tmp_path / "hand.gguf"
    p.write_bytes(head + b"\0" * (data_off - len(head)) + payload)
    g = gguf.GGUFFile(str(p))
    M = g.metadata
    assert g.version == 3 and g.data_offset == data_off
    assert (M["a.u8"].value, M["a.i8"].value, M["a.u16"].value, M["a.i16"].value) == (200, -5, 65000, -30000)
    assert (M["a.u32"].value, M["a.i32"].value, M["a.f32"].value, M["a.bool"].value) == (4000000000, -7, 1.5, True)
    assert M["a.str"].value == "héllo" and [v.value for v in M["tokenizer.ggml.tokens"].value] == ["x", "yy", "zzz"]
    assert [[w.value for w in v.value] for v in M["a.nested"].value] == [[1, 2], [3]]
    assert (M["a.u64"].value, M["a.i64"].value, M["a.f64"].value) == (2 ** 40 + 3, -2 ** 40, 0.1)
    # MetaValue::as_u32 wraps integer types (src/gguf.rs:131-141)
    assert g.get_u32("a.i32", 0) == (2 ** 32 - 7) and g.get_u32("a.u64", 0) == 3 and g.get_u32("a.f32", 9) == 9
    assert g.get_f32("a.f64", 0.0) == float(np.float32(0.1)) and g.get_f32("a.u32", 2.0) == 2.0
    t = g.tensors[0]
    assert (t.name, t.dims, t.dtype, t.offset, t.numel()) == ("t.weight", [32, 2], 8, 0, 64)
    assert bytes(g.tensor_bytes("t.weight")) == payload
    cfg = gguf.config_from_gguf(g)
    assert cfg["vocab"] == 3  # tokenizer.ggml.tokens length when no vocab_size
    # defaults of Config::from_gguf (src/model.rs:40-120)
    assert (cfg["max_seq_len"], cfg["eps"], cfg["theta"], cfg["window"]) == (2048, np.float32(1e-5), 10000.0, 0)
    g.close()


def test_bad_files_raise(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGU")
    with pytest.raises(ValueError, match="too small"):
        gguf.GGUFFile(str(p))
    p.write_bytes(b"GGML" + b"\0" * 32)
    with pytest.raises(ValueError, match="magic"):
        gguf.GGUFFile(str(p))
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + _s("k") + struct.pack("<I", 13))
    with pytest.raises(ValueError, match="value type 13"):
        gguf.GGUFFile(str(p))


def test_head_dim_override_from_shapes(tmp_path):
    """load_model prefers attn_q / attn_v shapes over misleading key_length /
    value_length metadata (src/model.rs:3668-3724)."""
    m = synth.make_model("tiny-q4km", seed=6)
    p = str(tmp_path / "hd.gguf")
    gguf.write_model(p, m)
    g = gguf.GGUFFile(p)
    md = []
    for k, v in g.metadata.items():
        if k.endswith("attention.key_length") or k.endswith("attention.value_length"):
            md.append((k, gguf.U32, 32))
        elif v.vtype == gguf.ARRAY:
            continue
        else:
            md.append((k, v.vtype, v.value))
    T = [(t.name, t.dims, t.dtype, g.tensor_bytes(t.name)) for t in g.tensors]
    p2 = str(tmp_path / "hd2.gguf")
    gguf.write(p2, md, T)
    g.close()
    g2 = gguf.GGUFFile(p2)
    assert gguf.config_from_gguf(g2)["head_dim"] == 32
    r = gguf.load_model(p2)
    assert r["config"]["head_dim"] == m["config"]["head_dim"] == 64 and r["config"]["value_dim"] == 64


@pytest.mark.parametrize("name,kw", [("tiny-q4km", {}), ("tiny-qwen", {}), ("tiny-q8", dict(tie_output=True,
                                                                                              fuse_qkv=True))])
def test_native_parser_agrees(tmp_path, name, kw):
    """The library's C++ parse (rusty_hip_gguf_summary, no GPU needed) reads
    the same header, config and layout facts as the Python reader."""
    from rustyllm_amd import hip
    m = synth.make_model(name, seed=8)
    p = str(tmp_path / "m.gguf")
    gguf.write_model(p, m, **kw)
    s = hip.gguf_summary(p)
    g = gguf.GGUFFile(p)
    c = gguf.config_from_gguf(g)
    assert s is not None and s.arch.decode() == c["arch"] and s.version == 3
    assert s.n_tensors == len(g.tensors) and s.data_offset == g.data_offset
    for k in ("n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "value_dim", "vocab"):
        assert getattr(s, k) == c[k], k
    assert s.hidden_dim == c["hidden_dim"] and s.context_length == c["max_seq_len"]
    assert np.float32(s.rope_theta) == np.float32(c["theta"]) and np.float32(s.rms_eps) == np.float32(c["eps"])
    assert s.tied_output == int(kw.get("tie_output", False)) and s.fused_qkv == int(kw.get("fuse_qkv", False))
    assert s.qkv_bias == int(bool(m["config"].get("qkv_bias")))


def test_native_parser_gptoss_and_hand_file(tmp_path):
    from rustyllm_amd import hip
    m = synth.make_gptoss("tiny-gptoss", seed=8)
    p = str(tmp_path / "g.gguf")
    gguf.write_model(p, m)
    s = hip.gguf_summary(p)
    c = m["config"]
    assert s.arch == b"gpt-oss" and (s.sliding_window, s.n_experts, s.top_k) == (c["window"], c["n_experts"],
                                                                                  c["top_k"])
    assert np.float32(s.rope_scaling) == np.float32(c["rope_scaling"]) and s.rope_orig_ctx == c["rope_orig_ctx"]
    test_parser_on_hand_built_bytes(tmp_path)
    s2 = hip.gguf_summary(str(tmp_path / "hand.gguf"))
    assert s2.data_offset % 64 == 0 and s2.vocab == 3 and s2.context_length == 2048 and s2.arch == b"llama"
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + _s("k") + struct.pack("<I", 13))
    assert hip.gguf_summary(str(bad)) is None
    bad.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 5))  # truncated metadata
    assert hip.gguf_summary(str(bad)) is None


def test_head_count_arrays_of_every_integer_type_and_corrupt_counts(tmp_path):
    """Config::from_gguf takes n_heads as the max over MetaValue::as_u32_array
    of a per-layer head_count array, which keeps non-negative signed entries
    (I8/I16 included) and drops negative ones and 64-bit values above
    u32::MAX (src/gguf.rs:188-207).  The vocabulary counts only the string
    entries of tokenizer.ggml.tokens (as_string_array, :161-176): an array of
    arrays counts none.  Both parsers agree.  Then counts that no file of this
    size could hold (metadata pairs, an array's length, tensor infos) are
    refused at once, with no allocation."""
    from rustyllm_amd import hip
    fmt = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 10: "Q", 11: "q"}
    cases = [(1, [-1, 40, 12], 40), (3, [-300, 36, 7], 36), (5, [-5, 24], 24), (11, [2 ** 33, -2, 30], 30),
             (10, [2 ** 33, 28], 28), (0, [200, 3], 200), (2, [1000, 9], 1000), (4, [4000000000, 1], 4000000000)]
    for et, vals, want in cases:
        arr = struct.pack("<IIQ", 9, et, len(vals)) + b"".join(struct.pack("<" + fmt[et], v) for v in vals)
        md = [_s("general.architecture") + struct.pack("<I", 8) + _s("llama"),
              _s("llama.embedding_length") + struct.pack("<II", 4, 4096),
              _s("llama.attention.head_count") + arr,
              _s("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, 3) + _s("a") + _s("bb") + _s("ccc")]
        p = tmp_path / f"hc{et}.gguf"
        p.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, len(md)) + b"".join(md) + b"\0" * 64)
        g = gguf.GGUFFile(str(p))
        c = gguf.config_from_gguf(g)
        g.close()
        assert c["n_heads"] == want and c["vocab"] == 3, (et, c["n_heads"])
        s = hip.gguf_summary(str(p))
        assert s is not None and s.n_heads == want and s.vocab == 3, (et, s.n_heads)
        assert s.head_dim == c["head_dim"] == 4096 // want
    # a token array whose entries are arrays (not strings) counts zero
    md2 = [_s("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 9, 2) + struct.pack("<IQ", 8, 1) + _s("x")
           + struct.pack("<IQ", 8, 1) + _s("y"), _s("llama.vocab_size") + struct.pack("<II", 4, 1)]
    p2 = tmp_path / "nested_tokens.gguf"
    p2.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, len(md2)) + b"".join(md2) + b"\0" * 64)
    g2 = gguf.GGUFFile(str(p2))
    assert gguf.config_from_gguf(g2)["vocab"] == 1
    g2.close()
    assert hip.gguf_summary(str(p2)).vocab == 1
    # counts far beyond what the file holds
    bad = tmp_path / "huge.gguf"
    bad.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 2 ** 60) + b"\0" * 256)
    assert hip.gguf_summary(str(bad)) is None
    bad.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 2 ** 50, 0) + b"\0" * 256)
    assert hip.gguf_summary(str(bad)) is None
    bad.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + _s("k") + struct.pack("<IIQ", 9, 8, 2 ** 40)
                    + b"\0" * 256)
    assert hip.gguf_summary(str(bad)) is None
    bad.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + _s("k") + struct.pack("<IIQ", 9, 10, 33)
                    + b"\0" * 256)  # 33 u64 entries need 264 bytes, 256 are left
    assert hip.gguf_summary(str(bad)) is None
