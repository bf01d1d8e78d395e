"""Pins the oracle's decode forward (forward_into, src/model.rs:7177-7358) and
decode loop (greedy + repeat penalty, src/runtime.rs:3266-3342) against an
independent float64 numpy restatement on small synthetic models."""
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
