"""gpt-oss decode on the device (the resident decoder in gpt-oss mode) against
the oracle's forward_gpt_oss_into (src/model.rs:6733-6908): Q8_0 attention
projections on f32 activations with biases, YaRN RoPE with its concentration,
attention with per-head sinks and a sliding window on even layers, wo + bo
on the Q8_K path, the routed MXFP4 MoE block, Q8_0 output head; greedy decode
with the reference's repeat penalty.  Every stage is in the reference's order,
so logits and KV are asserted bit-identical.
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


def test_gptoss_decode_logits_bit_exact(hip, exact):
    model = synth.make_gptoss("tiny-gptoss", seed=7)
    cfg = model["config"]
    res = hip.ResidentGptOss(model, 64)
    orc = O.OracleGptOss(model, 64)
    emb, et = model["token_embd"]
    dim = cfg["dim"]
    toks = synth.token_ids(11, 24, cfg["vocab"])  # 24 positions: past the 8-position window
    for pos, t in enumerate(toks):
        x = O.dequant_row(et, emb[int(t) * O.row_bytes(et, dim):], dim)
        g = res.decode(x, pos, 0, True)
        r = orc.forward(int(t), pos)
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), (pos, np.max(np.abs(g - r)))
    for layer in range(cfg["n_layers"]):
        assert np.array_equal(res.kv_read(layer, 0, 0, 24), orc.kc[layer][:24 * orc.kd])
        assert np.array_equal(res.kv_read(layer, 1, 0, 24), orc.vc[layer][:24 * orc.vdim])


def test_gptoss_greedy_stream(hip, exact):
    model = synth.make_gptoss("tiny-gptoss", seed=9)
    res = hip.ResidentGptOss(model, 80)
    orc = O.OracleGptOss(model, 80)
    prompt = synth.token_ids(4, 12, model["config"]["vocab"])
    g_toks, g_logits = res.generate(prompt, 24, penalty=1.1)
    o_toks, o_logits = orc.generate(prompt, 24, penalty=1.1)
    assert list(g_toks) == list(o_toks)
    assert np.array_equal(g_logits.view(np.uint32), o_logits.view(np.uint32))
