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

The prompt legs of configs 3 and 5 go through the batched prefill and are
checked against the oracle's sequential forward over the same prompt (the
reference prefills token by token: forward_prefill_batch against sequential
decode, src/model.rs:2877-2955; forward_prefill_gpt_oss per token,
src/runtime.rs:3760-3790):
- config 3: the 512-token prompt through the MFMA products at the 8B shape,
  KV of every layer and the next logits bit-exact;
- config 5: the 1024-token prompt at the 20B shape in two chunks (ring
  layers through the linear view), ring KV of every layer and the next
  logits bit-exact, then 64 greedy tokens.
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


_MODELS = {}


def _model(name, seed, gptoss=False):
    """One synthetic model per (name, seed) for the whole module: the 8B and
    20B shapes take tens of seconds to generate."""
    key = (name, seed)
    if key not in _MODELS:
        _MODELS.clear()  # hold one large model at a time
        _MODELS[key] = synth.make_gptoss(name, seed=seed) if gptoss else synth.make_model(name, seed=seed)
    return _MODELS[key]


def _standard_case(hip, name, ctx, n_steps, n_gen, seed):
    model = _model(name, seed)
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


def test_config3_llama3_8b_prompt_prefill_512(hip, exact):
    """BASELINE config 3's 512-token random prompt through the batched (MFMA)
    prefill at the 8B shape: every layer's K/V of the 511 prefilled
    positions and the next logits (the last prompt token's decode step)
    bit-identical to the oracle's token-by-token forward."""
    model = _model("llama3-8b-q4km", 1234)
    cfg = model["config"]
    n = 512
    storage = n + 16
    prompt = synth.token_ids(512, n, cfg["vocab"])
    res = hip.Resident(model, storage)
    _, g_logits = res.generate(prompt, 0)
    orc = O.OracleModel(model, storage, threads=16)
    for p, t in enumerate(prompt):
        o_logits = orc.forward(int(t), p, want_logits=p + 1 == n)
    assert np.array_equal(g_logits.view(np.uint32), o_logits.view(np.uint32)), np.max(np.abs(g_logits - o_logits))
    wk = cfg["n_kv_heads"] * cfg["head_dim"]
    wv = cfg["n_kv_heads"] * cfg["value_dim"]
    for layer in range(cfg["n_layers"]):
        ok, ov = orc.kv(layer, storage)
        assert np.array_equal(res.kv_read(layer, 0, 0, n).view(np.uint32), ok[: n * wk].view(np.uint32)), layer
        assert np.array_equal(res.kv_read(layer, 1, 0, n).view(np.uint32), ov[: n * wv].view(np.uint32)), layer
    del res, orc
    hip.weight_cache_clear()


def test_config4_qwen14b_ctx8192(hip, exact):
    _standard_case(hip, "qwen2.5-14b-q4km", 8192, 3, 4, seed=14)


def test_config4_qwen14b_ctx32768(hip, exact):
    _standard_case(hip, "qwen2.5-14b-q4km", 32768, 1, 8, seed=15)


def test_config5_gptoss20b_past_two_windows(hip, exact):
    model = _model("gpt-oss-20b", 20, gptoss=True)
    cfg = model["config"]
    max_len = 1024 + 256
    res = hip.ResidentGptOss(model, max_len)
    orc = O.OracleGptOss(model, max_len, threads=16)
    S = orc.storage
    assert S == 128 == res.slots
    _fill_kv(res, lambda l: (orc.kc[l], orc.vc[l]), cfg, S, 77)
    pos0 = 2 * S + 37  # every full layer walks the ring more than twice
    toks = synth.token_ids(20, 4, cfg["vocab"])
    _decode_steps(res, orc.forward, model, toks, pos0)
    for layer in (0, 1, cfg["n_layers"] - 1):
        assert np.array_equal(res.kv_read(layer, 0, 0, S), orc.kc[layer])
        assert np.array_equal(res.kv_read(layer, 1, 0, S), orc.vc[layer])
    # then 64 greedy tokens on the device against the oracle's decode loop
    pos = pos0 + len(toks)
    prompt = synth.token_ids(21, 2, cfg["vocab"])
    g_toks, g_logits = res.generate(prompt, 64, penalty=1.1, start_pos=pos)
    o_toks, o_logits = orc.generate(prompt, 64, penalty=1.1, start_pos=pos)
    assert list(g_toks) == list(o_toks)
    assert np.array_equal(g_logits.view(np.uint32), o_logits.view(np.uint32))
    del res, orc
    hip.weight_cache_clear()


def test_config5_gptoss20b_prompt_prefill_1024(hip, exact):
    """BASELINE config 5's 1024-token prompt at the gpt-oss-20B shape through
    the batched prefill (two chunks: 512 + 511 tokens, then the last token's
    decode step), against the reference's token-by-token prefill: the ring
    K/V of every layer and the next logits bit-identical, then the prompt
    again with 64 greedy tokens after it, identical to the oracle's decode
    loop continued from the same state."""
    model = _model("gpt-oss-20b", 20, gptoss=True)
    cfg = model["config"]
    n, n_gen = 1024, 64
    max_len = n + n_gen + 8
    prompt = synth.token_ids(1024, n, cfg["vocab"])
    res = hip.ResidentGptOss(model, max_len)
    S = res.slots
    _, g_logits = res.generate(prompt, 0)
    orc = O.OracleGptOss(model, max_len, threads=16)
    assert orc.storage == S == cfg["window"]
    for p, t in enumerate(prompt):
        o_logits = orc.forward(int(t), p, want_logits=p + 1 == n)
        if p % 256 == 255:
            print(f"[config5 prefill] oracle at position {p + 1}/{n}", flush=True)
    assert np.array_equal(g_logits.view(np.uint32), o_logits.view(np.uint32)), np.max(np.abs(g_logits - o_logits))
    for layer in range(cfg["n_layers"]):
        assert np.array_equal(res.kv_read(layer, 0, 0, S).view(np.uint32), orc.kc[layer].view(np.uint32)), layer
        assert np.array_equal(res.kv_read(layer, 1, 0, S).view(np.uint32), orc.vc[layer].view(np.uint32)), layer
    # the decode loop after the prompt (runtime.rs:3266-3342): the device
    # prefills the prompt again and generates; the oracle continues from its
    # state with the prompt's last 64 tokens as the penalty window
    g_toks, g_last = res.generate(prompt, n_gen, penalty=1.1)
    recent = [int(t) for t in prompt[-64:]]
    logits, pos, o_toks = o_logits, n, []
    for i in range(n_gen):
        o_last = logits
        tok, _ = O.greedy(logits, recent, 1.1)
        o_toks.append(tok)
        recent = (recent + [tok])[-64:]
        if i + 1 < n_gen:
            logits = orc.forward(tok, pos)
            pos += 1
    assert list(g_toks) == o_toks
    assert np.array_equal(g_last.view(np.uint32), o_last.view(np.uint32))
    del res, orc
    hip.weight_cache_clear()


def test_config5_gptoss20b_expert_mfma_stream(hip, exact):
    """The opt-in matrix-core expert product (rusty_hip_set_expert_mfma) at
    the gpt-oss-20B shape: config 5's 1024-token prompt prefilled with it, then
    64 greedy tokens, against the same run with the reference's serial sums
    (the stream the test above pins to the oracle).  After a 16-token prompt
    the first layer's K (computed before any expert product) is identical and
    the second layer's (through f32 paths from the first layer's products)
    within a relative 1e-5; the difference in later layers, in the logits
    after longer prompts, and how many greedy tokens agree are printed: the
    int8 (Q8_K) activation of wo and the top-k routing turn rounding-level
    differences into whole quantization steps and expert flips, so the
    difference grows through the layers."""
    model = _model("gpt-oss-20b", 20, gptoss=True)
    cfg = model["config"]
    n, n_gen = 1024, 64
    prompt = synth.token_ids(1024, n, cfg["vocab"])
    res = hip.ResidentGptOss(model, n + n_gen + 8)
    prev = hip.set_expert_mfma(False)
    growth, layers = [], []
    try:
        # where the difference enters: the K/V of every layer after a 16-token
        # prompt (layer 0's come before any expert product, layer 1's from the
        # first layer's products through f32 paths only); then how it grows
        # with the prompt's length
        kv = []
        for on in (False, True):
            hip.set_expert_mfma(on)
            assert res.prefill(prompt[:16], 0)
            kv.append([res.kv_read(layer, 0, 0, 16) for layer in range(cfg["n_layers"])])
        for layer in range(cfg["n_layers"]):
            a, b = kv[0][layer], kv[1][layer]
            layers.append(float(np.max(np.abs(b - a)) / np.max(np.abs(a))))
        for m in (16, 128, 512):
            hip.set_expert_mfma(False)
            _, a = res.generate(prompt[:m], 0)
            hip.set_expert_mfma(True)
            _, b = res.generate(prompt[:m], 0)
            growth.append((m, float(np.max(np.abs(b - a)) / np.max(np.abs(a)))))
        hip.set_expert_mfma(False)
        _, e_logits = res.generate(prompt, 0)
        e_toks, _ = res.generate(prompt, n_gen, penalty=1.1)
        hip.set_expert_mfma(True)
        _, m_logits = res.generate(prompt, 0)
        m_toks, _ = res.generate(prompt, n_gen, penalty=1.1)
    finally:
        hip.set_expert_mfma(prev)
    rel = float(np.max(np.abs(m_logits - e_logits)) / np.max(np.abs(e_logits)))
    print("[config5 expert mfma] relative K difference by layer after 16 tokens: " +
          ", ".join(f"{r:.2g}" for r in layers), flush=True)
    print("[config5 expert mfma] relative logit difference by prompt length: " +
          ", ".join(f"{m}: {r:.3g}" for m, r in growth + [(n, rel)]), flush=True)
    e_toks, m_toks = list(e_toks), list(m_toks)
    same = sum(int(a == b) for a, b in zip(e_toks, m_toks))
    prefix = next((i for i, (a, b) in enumerate(zip(e_toks, m_toks)) if a != b), len(e_toks))
    print(f"[config5 expert mfma] logits after the prompt: max relative difference {rel:.3g}; greedy tokens "
          f"equal {same}/{n_gen}, identical prefix {prefix}", flush=True)
    assert layers[0] == 0.0 and layers[1] <= 1e-5, layers
    del res
    hip.weight_cache_clear()
