"""End-to-end decode parity at the BASELINE.json model shapes (configs 3-5),
the resident HIP decoder against the oracle on the same synthetic model.

The long contexts are filled the way bench.py's profiler runs fill them: the
same N(0, 1) K/V rows written to both caches (positions 0..ctx-2), so the
decode steps that follow attend over a full context without a 4K-token
prompt on the CPU side.  Then several decode steps (host embedding, logits
every step) and a greedy continuation on the device are compared bit for
bit: logits, K/V of the new positions and tokens.

- config 3, Llama-3-8B Q4_K_M at ctx 4096: the transposed-V chain path at a
  4K range, the 14336-row SwiGLU tiles, the RMSNorm-prologue 128256-row head,
  and a 64-token greedy stream (the north star's bar);
- config 4, Qwen2.5-14B at ctx 8192 and one step at 32768: d_model 5120
  (K = 5120 activations), 40 q / 8 kv heads (kv_mul 5, the per-head update
  form), NeoX RoPE, QKV biases;
- config 5, gpt-oss-20B past two ring lengths: the 128-slot window ring
  scanned cyclically by the full layers, sinks, MXFP4 experts, 201088-row
  Q8_0 head on f32 activations, then a 24-token greedy stream.
"""
import numpy as np
import pytest

from oracle import oracle as O
from rustyllm_amd import synth

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]


@pytest.fixture
def exact(hip):
    prev = hip.attention_mode("exact")
    yield
    hip.attention_mode(prev)


def _fill_kv(res, orc_kv, cfg, n_slots, seed):
    """Same N(0,1) rows into both caches, slots 0..n_slots-1, layer by layer."""
    wk = cfg["n_kv_heads"] * cfg["head_dim"]
    wv = cfg["n_kv_heads"] * cfg["value_dim"]
    for layer in range(cfg["n_layers"]):
        ok, ov = orc_kv(layer)
        for which, w, dst in ((0, wk, ok), (1, wv, ov)):
            data = synth.normal_f32(seed + 2 * layer + which, n_slots, w, 1.0).reshape(-1)
            res.kv_write(layer, which, 0, data)
            dst[: data.size] = data


def _decode_steps(res, orc_forward, model, toks, pos0):
    emb, et = model["token_embd"]
    dim = model["config"]["dim"]
    for i, t in enumerate(toks):
        x = O.dequant_row(et, emb[int(t) * O.row_bytes(et, dim):], dim)
        g = res.decode(x, pos0 + i, 0, True)
        r = orc_forward(int(t), pos0 + i)
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), (pos0 + i, np.max(np.abs(g - r)))


def _standard_case(hip, name, ctx, n_steps, n_gen, seed):
    model = synth.make_model(name, seed=seed)
    cfg = model["config"]
    storage = ctx + n_steps + n_gen + 8
    res = hip.Resident(model, storage)
    orc = O.OracleModel(model, storage, threads=16)
    _fill_kv(res, lambda l: orc.kv(l, storage), cfg, ctx - 1, seed * 31)
    toks = synth.token_ids(seed, n_steps + 1, cfg["vocab"])
    _decode_steps(res, orc.forward, model, toks[:n_steps], ctx - 1)
    pos = ctx - 1 + n_steps
    for layer in (0, cfg["n_layers"] - 1):
        for which in (0, 1):
            ok, ov = orc.kv(layer, storage)
            w = cfg["n_kv_heads"] * (cfg["value_dim"] if which else cfg["head_dim"])
            ref = (ov if which else ok)[(ctx - 1) * w: pos * w]
            assert np.array_equal(res.kv_read(layer, which, ctx - 1, n_steps), ref)
    if n_gen:
        g_toks, g_logits = res.generate(toks[n_steps:], n_gen, penalty=1.1, start_pos=pos)
        o_toks, o_logits = orc.generate(toks[n_steps:], n_gen, penalty=1.1, start_pos=pos)
        assert list(g_toks) == list(o_toks)
        assert np.array_equal(g_logits.view(np.uint32), o_logits.view(np.uint32))
    del res, orc
    hip.weight_cache_clear()


def test_config3_llama3_8b_ctx4096(hip, exact):
    # the north star's bar: the greedy stream identical for the first 64 tokens
    _standard_case(hip, "llama3-8b-q4km", 4096, 4, 64, seed=1234)


def test_config4_qwen14b_ctx8192(hip, exact):
    _standard_case(hip, "qwen2.5-14b-q4km", 8192, 3, 4, seed=14)


def test_config4_qwen14b_ctx32768(hip, exact):
    _standard_case(hip, "qwen2.5-14b-q4km", 32768, 1, 0, seed=15)


def test_config5_gptoss20b_past_two_windows(hip, exact):
    model = synth.make_gptoss("gpt-oss-20b", seed=20)
    cfg = model["config"]
    max_len = 1024 + 256
    res = hip.ResidentGptOss(model, max_len)
    orc = O.OracleGptOss(model, max_len)
    S = orc.storage
    assert S == 128 == res.slots
    _fill_kv(res, lambda l: (orc.kc[l], orc.vc[l]), cfg, S, 77)
    pos0 = 2 * S + 37  # every full layer walks the ring more than twice
    toks = synth.token_ids(20, 4, cfg["vocab"])
    _decode_steps(res, orc.forward, model, toks, pos0)
    for layer in (0, 1, cfg["n_layers"] - 1):
        assert np.array_equal(res.kv_read(layer, 0, 0, S), orc.kc[layer])
        assert np.array_equal(res.kv_read(layer, 1, 0, S), orc.vc[layer])
    # then 24 greedy tokens on the device against the oracle's decode loop
    # (the oracle composes this model's layers in Python, ~1.2 s per token)
    pos = pos0 + len(toks)
    prompt = synth.token_ids(21, 2, cfg["vocab"])
    g_toks, g_logits = res.generate(prompt, 24, penalty=1.1, start_pos=pos)
    o_toks, o_logits = orc.generate(prompt, 24, penalty=1.1, start_pos=pos)
    assert list(g_toks) == list(o_toks)
    assert np.array_equal(g_logits.view(np.uint32), o_logits.view(np.uint32))
