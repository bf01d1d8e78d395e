"""bf16 KV cache on the device (rusty_hip_resident_enable_bf16: the
reference's KVCache::enable_bf16, src/model.rs:1406-1421, with
attention_over_kv_heads_bf16, :6205-6580) against the oracle's bf16 cache:
stored K/V bit patterns, logits and greedy streams bit-identical, through
the decode step, the batched prefill and an unaligned attention start (the
widened-row fallback)."""
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


def _pair(hip, name, storage, seed):
    model = synth.make_model(name, seed=seed)
    return (model, hip.Resident(model, storage, kv_bf16=True),
            O.OracleModel(model, storage, threads=16, kv_bf16=True))


@pytest.mark.parametrize("name", ["tiny-q4km", "tiny-q8", "tiny-qwen"])
def test_bf16_decode_bit_exact(hip, exact, name):
    model, res, orc = _pair(hip, name, 96, 11)
    emb, et = model["token_embd"]
    dim = model["config"]["dim"]
    toks = synth.token_ids(3, 80, model["config"]["vocab"])
    for pos, t in enumerate(toks):
        x = O.dequant_row(et, emb[int(t) * O.row_bytes(et, dim):], dim)
        g = res.decode(x, pos, 0, True)
        r = orc.forward(int(t), pos)
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), (pos, np.max(np.abs(g - r)))
    for layer in range(model["config"]["n_layers"]):
        for which in (0, 1):
            gk = res.kv_read(layer, which, 0, 80)
            ok, ov = orc.kv(layer, 96)
            assert gk.dtype == np.uint16 and np.array_equal(gk, (ov if which else ok)[: gk.size])


@pytest.mark.parametrize("name,penalty", [("tiny-q4km", 1.1), ("tiny-qwen", 1.0)])
def test_bf16_greedy_stream_with_batched_prefill(hip, exact, name, penalty):
    model, res, orc = _pair(hip, name, 200, 12)
    prompt = synth.token_ids(21, 100, model["config"]["vocab"])
    g_toks, g_logits = res.generate(prompt, 64, penalty=penalty)
    o_toks, o_logits = orc.generate(prompt, 64, penalty=penalty)
    assert list(g_toks) == list(o_toks)
    assert np.array_equal(g_logits.view(np.uint32), o_logits.view(np.uint32))


def test_bf16_unaligned_start_and_mode_switch(hip, exact):
    """An attention start that is not a multiple of 4 positions takes the
    widened-row fallback; switching the cache back to f32 gives the f32
    decoder again."""
    model, res, orc = _pair(hip, "tiny-qwen", 96, 13)
    emb, et = model["token_embd"]
    dim = model["config"]["dim"]
    toks = synth.token_ids(4, 70, model["config"]["vocab"])
    for pos, t in enumerate(toks):
        st = 0 if pos < 8 else (pos // 3) | 1
        x = O.dequant_row(et, emb[int(t) * O.row_bytes(et, dim):], dim)
        g = res.decode(x, pos, st, True)
        r = orc.forward(int(t), pos, start_t=st)
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), (pos, st)
    res.enable_bf16(False)
    orc32 = O.OracleModel(model, 96, threads=16)
    for pos, t in enumerate(toks[:20]):
        x = O.dequant_row(et, emb[int(t) * O.row_bytes(et, dim):], dim)
        assert np.array_equal(res.decode(x, pos, 0, True), orc32.forward(int(t), pos))
