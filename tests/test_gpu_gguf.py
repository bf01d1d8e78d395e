"""The GGUF on-disk path on the device: a synthetic model written to a GGUF
v3 file (rustyllm_amd.gguf.write_model), loaded by the library itself
(rusty_hip_resident_load_gguf: native parse, tensor mapping as the
reference's load_model / load_gpt_oss_model, pinned-staged upload), then
decoded against the oracle built on the same file's bytes: logits, KV and
greedy streams bit-identical.  Covers the tied output head, the fused
attn_qkv split and the gpt-oss ring."""
import numpy as np
import pytest

from oracle import oracle as O
from rustyllm_amd import gguf, synth

pytestmark = pytest.mark.gpu


@pytest.fixture
def exact(hip):
    prev = hip.attention_mode("exact")
    yield
    hip.attention_mode(prev)


@pytest.mark.parametrize("name,kw", [("tiny-q4km", {}), ("tiny-qwen", {}),
                                     ("tiny-q8", dict(tie_output=True, fuse_qkv=True))])
def test_standard_model_from_gguf(hip, exact, tmp_path, name, kw):
    m = synth.make_model(name, seed=21)
    p = str(tmp_path / f"{name}.gguf")
    gguf.write_model(p, m, **kw)
    res = hip.ResidentGguf(p, 96)
    fm = gguf.load_model(p)
    orc = O.OracleModel(fm, 96, threads=8)
    prompt = synth.token_ids(2, 20, m["config"]["vocab"])
    g_toks, g_logits = res.generate(prompt, 40, penalty=1.1)
    o_toks, o_logits = orc.generate(prompt, 40, penalty=1.1)
    assert list(g_toks) == list(o_toks)
    assert np.array_equal(g_logits.view(np.uint32), o_logits.view(np.uint32))
    # the same decode from the in-memory model gives the same bits (a tied
    # file has no output.weight: its head is the embedding table)
    if kw.get("tie_output"):
        m = dict(m, output=m["token_embd"])
    orc2 = O.OracleModel(m, 96, threads=8)
    t2, l2 = orc2.generate(prompt, 40, penalty=1.1)
    assert list(t2) == list(o_toks) and np.array_equal(l2, o_logits)
    ok, ov = orc.kv(0, 96)
    n = len(prompt) + 39
    assert np.array_equal(res.kv_read(0, 0, 0, n), ok[: n * m["config"]["n_kv_heads"] * m["config"]["head_dim"]])


def test_gptoss_from_gguf(hip, exact, tmp_path):
    m = synth.make_gptoss("tiny-gptoss-w128", seed=22)
    p = str(tmp_path / "gptoss.gguf")
    gguf.write_model(p, m)
    res = hip.ResidentGguf(p, 512)
    assert res.summary.sliding_window == 128
    fm = gguf.load_model(p)
    orc = O.OracleGptOss(fm, 512)
    prompt = synth.token_ids(3, 150, m["config"]["vocab"])
    g_toks, g_logits = res.generate(prompt, 140, penalty=1.1)
    o_toks, o_logits = orc.generate(prompt, 140, penalty=1.1)
    assert list(g_toks) == list(o_toks)
    assert np.array_equal(g_logits.view(np.uint32), o_logits.view(np.uint32))


def test_load_gguf_rejects_bad_files(hip, tmp_path):
    p = tmp_path / "x.gguf"
    p.write_bytes(b"not a gguf file at all")
    assert hip.lib.rusty_hip_resident_load_gguf(str(p).encode(), 64) == 0
    m = synth.make_model("tiny-q4km", seed=1)
    q = str(tmp_path / "ok.gguf")
    gguf.write_model(q, m)
    assert hip.lib.rusty_hip_resident_load_gguf(q.encode(), 0) == 0
    data = open(q, "rb").read()
    trunc = tmp_path / "trunc.gguf"
    trunc.write_bytes(data[: len(data) // 2])  # tensors run past the end of the file
    assert hip.lib.rusty_hip_resident_load_gguf(str(trunc).encode(), 64) == 0
