"""Pins the oracle's decode forward (forward_into, src/model.rs:7177-7358) and
decode loop (greedy + repeat penalty, src/runtime.rs:3266-3342) against an
independent float64 numpy restatement on small synthetic models."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from rustyllm_amd import synth
from tests import npref


@pytest.mark.parametrize("name", ["tiny-q4km", "tiny-q8", "tiny-qwen"])
def test_forward_logits_vs_f64(name):
    model = synth.make_model(name, seed=3)
    toks = [int(t) for t in synth.token_ids(5, 6, model["config"]["vocab"])]
    om = O.OracleModel(model, storage_len=32, threads=4)
    got = np.array([om.forward(t, p) for p, t in enumerate(toks)])
    ref = npref.forward_model(model, toks)
    scale = np.abs(ref).max()
    # int8 activation rounding can flip by one quantum between f32 and f64
    # intermediates; orchestration mistakes show up at O(scale).
    assert np.max(np.abs(got - ref)) < 5e-4 * scale, (np.max(np.abs(got - ref)), scale)


def test_generate_matches_manual_loop():
    model = synth.make_model("tiny-q4km", seed=4)
    vocab = model["config"]["vocab"]
    prompt = synth.token_ids(9, 5, vocab)
    a = O.OracleModel(model, storage_len=64, threads=2)
    toks, _ = a.generate(prompt, 12, penalty=1.1)
    b = O.OracleModel(model, storage_len=64, threads=2)
    recent = list(prompt[-64:])
    logits = None
    for p, t in enumerate(prompt):
        logits = b.forward(int(t), p)
    manual = []
    pos = len(prompt)
    for g in range(12):
        tok, _ = O.greedy(logits, recent, 1.1)
        manual.append(tok)
        recent = (recent + [tok])[-64:]
        if g + 1 < 12:
            logits = b.forward(tok, pos)
            pos += 1
    assert list(toks) == manual


def test_gptoss_forward_vs_f64_with_ring():
    """OracleGptOss (forward_gpt_oss_into with the reference's window-sized KV
    ring) against the float64 restatement, past three ring lengths: the odd
    layers then scan the ring from slot 0 cyclically (pos + 1 steps)."""
    model = synth.make_gptoss("tiny-gptoss", seed=5)
    c = model["config"]
    W = c["window"]
    n = 3 * W + 5
    toks = [int(t) for t in synth.token_ids(17, n, c["vocab"])]
    orc = O.OracleGptOss(model, 64)
    assert orc.storage == W and orc.ring
    got = np.array([orc.forward(t, p) for p, t in enumerate(toks)])
    ref = npref.forward_gptoss(model, toks, 64)
    scale = np.abs(ref).max()
    assert np.max(np.abs(got - ref)) < 5e-4 * scale, (np.max(np.abs(got - ref)), scale)
    # the check is sensitive to the ring: a linear cache agrees up to the
    # first wrap and then departs by far more than the tolerance
    lin = npref.forward_gptoss(model, toks, 64, ring=False)
    assert np.max(np.abs(lin[:W] - ref[:W])) < 1e-9 * scale
    assert np.max(np.abs(lin[W + 1:] - ref[W + 1:])) > 1e-2 * scale


def test_gptoss_c_layer_loop_equals_composed():
    """The C layer loop (orc_gptoss_forward) against the same forward composed
    step by step in Python from the C parts (router, experts, sinks, ring):
    logits, prefill steps without the head, and every layer's ring KV
    bit-identical past three ring lengths.  The composed form is the one the
    float64 checks above pin; this carries that pin over to the C loop."""
    model = synth.make_gptoss("tiny-gptoss", seed=9)
    c = model["config"]
    n = 3 * c["window"] + 7
    toks = [int(t) for t in synth.token_ids(23, n, c["vocab"])]
    a = O.OracleGptOss(model, 64, threads=4)
    b = O.OracleGptOssComposed(model, 64)
    for p, t in enumerate(toks):
        la = a.forward(t, p, want_logits=p % 5 != 3)
        lb = b.forward(t, p)
        if p % 5 != 3:
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), p
    for l in range(c["n_layers"]):
        assert np.array_equal(a.kc[l].view(np.uint32), b.kc[l].view(np.uint32)), l
        assert np.array_equal(a.vc[l].view(np.uint32), b.vc[l].view(np.uint32)), l
    ta, la = a.generate(toks[:9], 6, penalty=1.1, start_pos=n)
    tb, lb = b.generate(toks[:9], 6, penalty=1.1, start_pos=n)
    assert list(ta) == list(tb) and np.array_equal(la.view(np.uint32), lb.view(np.uint32))


def test_gptoss_reference_schedule_same_values():
    """The CPU baseline times the oracle on the reference's own schedule (one
    MXFP4 row per scalar dot, sink heads one after another); the checker's
    faster schedule must give the same bits."""
    model = synth.make_gptoss("tiny-gptoss", seed=3)
    toks = [int(t) for t in synth.token_ids(5, 30, model["config"]["vocab"])]
    a = O.OracleGptOss(model, 64, threads=4)
    la = [a.forward(t, p) for p, t in enumerate(toks)]
    O.lib.orc_set_fast_schedule(0)
    try:
        b = O.OracleGptOss(model, 64, threads=4)
        lb = [b.forward(t, p) for p, t in enumerate(toks)]
    finally:
        O.lib.orc_set_fast_schedule(1)
    for x, y in zip(la, lb):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


def test_gptoss_short_cache_is_linear():
    """max_len below the window: storage_len_for gives max_len slots and no
    position ever wraps."""
    model = synth.make_gptoss("tiny-gptoss", seed=6)
    c = model["config"]
    toks = [int(t) for t in synth.token_ids(3, 6, c["vocab"])]
    orc = O.OracleGptOss(model, 6)
    assert orc.storage == 6
    got = np.array([orc.forward(t, p) for p, t in enumerate(toks)])
    ref = npref.forward_gptoss(model, toks, 6)
    assert np.max(np.abs(got - ref)) < 5e-4 * np.abs(ref).max()


@pytest.mark.parametrize("theta,hd,scaling,orig", [(150000.0, 64, 32.0, 4096), (10000.0, 128, 4.0, 8192),
                                                   (150000.0, 64, 1.0, 4096)])
def test_yarn_table(theta, hd, scaling, orig):
    """build_rope_inv_freq_gpt_oss (model.rs:3059-3098): the synthetic model's
    table (csrc/synth.cpp) equals the oracle's bit for bit, and the oracle is
    pinned by the ramp's closed form: pairs below `low` keep 1/base, pairs
    above `high` get 1/(scaling*base) (both exactly, in f32), the ramp in
    between within 1e-6 of float64, the concentration 0.1 ln(s) + 1."""
    inv, conc = O.rope_inv_freq_gpt_oss(theta, hd, scaling, orig)
    s_inv, s_conc = synth.rope_gpt_oss(theta, hd, scaling, orig)
    assert np.array_equal(inv.view(np.uint32), s_inv.view(np.uint32)) and conc == s_conc
    f = np.float32
    # libm powf itself (numpy's float32 power can differ from it in the last bit)
    libm = ctypes.CDLL("libm.so.6")
    libm.powf.restype = ctypes.c_float
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    base = np.array([libm.powf(theta, float(f(2 * i) / f(hd))) for i in range(hd // 2)], np.float32)
    if scaling <= 1.0:
        assert conc == 1.0
        assert np.array_equal(inv, (f(1.0) / base).astype(np.float32))
        assert np.array_equal(inv, O.rope_inv_freq(theta, hd, 1.0))
        return
    assert abs(conc - (0.1 * np.log(scaling) + 1.0)) < 1e-6
    half = hd / 2
    low = half * np.log(orig / (32 * 2 * np.pi)) / np.log(theta)
    high = half * np.log(orig / (2 * np.pi)) / np.log(theta)
    b64 = np.power(np.float64(theta), np.arange(hd // 2) * 2.0 / hd)
    ramp = np.clip((np.arange(hd // 2) - low) / (high - low), 0.0, 1.0)
    ref = (1.0 / (scaling * b64)) * ramp + (1.0 / b64) * (1.0 - ramp)
    assert np.max(np.abs(inv - ref) / ref) < 1e-5
    lo_pairs = np.arange(hd // 2) < np.floor(low) - 1
    hi_pairs = np.arange(hd // 2) > np.ceil(high) + 1
    assert lo_pairs.any() and hi_pairs.any()
    assert np.array_equal(inv[lo_pairs], (f(1.0) / base[lo_pairs]).astype(np.float32))
    assert np.array_equal(inv[hi_pairs], (f(1.0) / (f(scaling) * base[hi_pairs])).astype(np.float32))
    assert np.all(np.diff(inv) < 0)


@pytest.mark.parametrize("name", ["tiny-q4km", "tiny-qwen"])
def test_forward_bf16_kv_vs_f64(name):
    """forward_into with KVCache::enable_bf16 (the oracle's bf16 cache and
    attention_over_kv_heads_bf16) against the float64 forward whose cache
    holds bf16-rounded K/V; the same bound as the f32 cache."""
    model = synth.make_model(name, seed=3)
    toks = [int(t) for t in synth.token_ids(5, 6, model["config"]["vocab"])]
    om = O.OracleModel(model, storage_len=32, threads=4, kv_bf16=True)
    got = np.array([om.forward(t, p) for p, t in enumerate(toks)])
    ref = npref.forward_model(model, toks, kv_bf16=True)
    scale = np.abs(ref).max()
    assert np.max(np.abs(got - ref)) < 5e-4 * scale, (np.max(np.abs(got - ref)), scale)
    k, v = om.kv(0, 32)
    assert k.dtype == np.uint16 and np.any(k[: 6 * model["config"]["n_kv_heads"] * 64] != 0)
