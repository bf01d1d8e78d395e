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
