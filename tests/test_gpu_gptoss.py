"""gpt-oss decode on the device (the resident decoder in gpt-oss mode) against
the oracle's forward_gpt_oss_into (src/model.rs:6733-6908): Q8_0 attention
projections on f32 activations with biases, YaRN RoPE with its concentration,
the KV cache as the reference's window-sized ring (min(window, max_len) slots,
slot = pos % slots, src/model.rs:1450-1464), attention with per-head sinks
over that ring (sliding window on even layers, the full layers scanning from
position 0 and so revisiting slots once pos >= slots), wo + bo on the Q8_K
path, the routed MXFP4 MoE block, Q8_0 output head; greedy decode with the
reference's repeat penalty.  Every stage is in the reference's order, so
logits and KV are asserted bit-identical.

Window 8 runs the small-ring attention kernels (a ring shorter than one
64-position tile); window 128 the LDS-tiled ones.  Both go past three ring
lengths.
"""
import numpy as np
import pytest

from oracle import oracle as O
from rustyllm_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture
def exact(hip):
    prev = hip.attention_mode("exact")
    yield
    hip.attention_mode(prev)


@pytest.mark.parametrize("name,max_len,n", [("tiny-gptoss", 64, 30), ("tiny-gptoss-w128", 512, 400)])
def test_gptoss_decode_logits_bit_exact(hip, exact, name, max_len, n):
    model = synth.make_gptoss(name, seed=7)
    cfg = model["config"]
    res = hip.ResidentGptOss(model, max_len)
    orc = O.OracleGptOss(model, max_len)
    assert orc.storage == cfg["window"] and n >= 3 * orc.storage
    emb, et = model["token_embd"]
    dim = cfg["dim"]
    toks = synth.token_ids(11, n, cfg["vocab"])
    for pos, t in enumerate(toks):
        x = O.dequant_row(et, emb[int(t) * O.row_bytes(et, dim):], dim)
        g = res.decode(x, pos, 0, True)
        r = orc.forward(int(t), pos)
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), (pos, np.max(np.abs(g - r)))
    S = orc.storage
    for layer in range(cfg["n_layers"]):
        assert np.array_equal(res.kv_read(layer, 0, 0, S), orc.kc[layer])
        assert np.array_equal(res.kv_read(layer, 1, 0, S), orc.vc[layer])
    # the ring has exactly `window` slots: one more is out of range
    with pytest.raises(RuntimeError):
        res.kv_read(0, 0, 0, S + 1)


@pytest.mark.parametrize("name,max_len,n_prompt,n_gen", [("tiny-gptoss", 80, 12, 24),
                                                         ("tiny-gptoss-w128", 512, 300, 100)])
def test_gptoss_greedy_stream(hip, exact, name, max_len, n_prompt, n_gen):
    model = synth.make_gptoss(name, seed=9)
    res = hip.ResidentGptOss(model, max_len)
    orc = O.OracleGptOss(model, max_len)
    prompt = synth.token_ids(4, n_prompt, model["config"]["vocab"])
    g_toks, g_logits = res.generate(prompt, n_gen, penalty=1.1)
    o_toks, o_logits = orc.generate(prompt, n_gen, penalty=1.1)
    assert list(g_toks) == list(o_toks)
    assert np.array_equal(g_logits.view(np.uint32), o_logits.view(np.uint32))


@pytest.mark.parametrize("name,max_len,pieces", [
    ("tiny-gptoss", 80, [(0, 30), (30, 61)]),           # ring of 8: every chunk wraps it many times
    ("tiny-gptoss-w128", 512, [(0, 200), (200, 390)]),  # ring of 128: chunks longer than the ring
])
def test_gptoss_prefill_kv_and_next_logits_bit_exact(hip, exact, name, max_len, pieces):
    """Batched gpt-oss prefill (the reference prefills gpt-oss token by token,
    forward_prefill_gpt_oss): after prefilling the prompt in pieces, the ring
    K/V of every layer and the next decode step's logits equal the oracle's
    sequential forward bit for bit.  Each token attends the ring as it stood
    at its own step, also across the pieces."""
    model = synth.make_gptoss(name, seed=13)
    cfg = model["config"]
    res = hip.ResidentGptOss(model, max_len)
    orc = O.OracleGptOss(model, max_len)
    n = pieces[-1][1]
    toks = synth.token_ids(21, n + 1, cfg["vocab"])
    for a, b in pieces:
        assert res.prefill(toks[a:b], a)
    for pos in range(n):
        orc.forward(int(toks[pos]), pos)
    S = orc.storage
    for layer in range(cfg["n_layers"]):
        assert np.array_equal(res.kv_read(layer, 0, 0, S).view(np.uint32), orc.kc[layer].view(np.uint32)), layer
        assert np.array_equal(res.kv_read(layer, 1, 0, S).view(np.uint32), orc.vc[layer].view(np.uint32)), layer
    emb, et = model["token_embd"]
    x = O.dequant_row(et, emb[int(toks[n]) * O.row_bytes(et, cfg["dim"]):], cfg["dim"])
    g = res.decode(x, n, 0, True)
    r = orc.forward(int(toks[n]), n)
    assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), np.max(np.abs(g - r))


def test_gptoss_prefill_after_decoded_positions(hip, exact):
    """Prefill that continues a ring the decode step started, then decode."""
    model = synth.make_gptoss("tiny-gptoss", seed=5)
    cfg = model["config"]
    res = hip.ResidentGptOss(model, 64)
    orc = O.OracleGptOss(model, 64)
    toks = synth.token_ids(8, 40, cfg["vocab"])
    emb, et = model["token_embd"]
    dim = cfg["dim"]

    def x_of(t):
        return O.dequant_row(et, emb[int(t) * O.row_bytes(et, dim):], dim)

    for pos in range(5):
        res.decode(x_of(toks[pos]), pos, 0, False)
    assert res.prefill(toks[5:33], 5)
    for pos in range(33):
        orc.forward(int(toks[pos]), pos)
    for pos in range(33, 40):
        g = res.decode(x_of(toks[pos]), pos, 0, True)
        r = orc.forward(int(toks[pos]), pos)
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), pos


def test_gptoss_prefill_q8k_widths(hip, exact):
    """A gpt-oss shape whose d_model is a multiple of 256: the attention
    projections and the router then take the Q8_K integer path (the decode
    step's Q8_0 x Q8_K kernels), batched over the chunk's tokens."""
    cfg = dict(synth.GPTOSS_CONFIGS["tiny-gptoss-w128"], dim=256, n_heads=4, head_dim=64, window=16)
    model = synth.make_gptoss(cfg, seed=17)
    res = hip.ResidentGptOss(model, 96)
    orc = O.OracleGptOss(model, 96)
    n = 70
    toks = synth.token_ids(3, n + 1, cfg["vocab"])
    assert res.prefill(toks[:40], 0) and res.prefill(toks[40:n], 40)
    for pos in range(n):
        orc.forward(int(toks[pos]), pos)
    S = orc.storage
    for layer in range(cfg["n_layers"]):
        assert np.array_equal(res.kv_read(layer, 0, 0, S).view(np.uint32), orc.kc[layer].view(np.uint32)), layer
        assert np.array_equal(res.kv_read(layer, 1, 0, S).view(np.uint32), orc.vc[layer].view(np.uint32)), layer
    emb, et = model["token_embd"]
    x = O.dequant_row(et, emb[int(toks[n]) * O.row_bytes(et, cfg["dim"]):], cfg["dim"])
    g = res.decode(x, n, 0, True)
    r = orc.forward(int(toks[n]), n)
    assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), np.max(np.abs(g - r))
