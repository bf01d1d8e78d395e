"""GPU parity of the batched (prefill) path against the oracle, through the
C ABI of librusty_hip.so.

The batched K-quant product (matvec_kquant_batch_into, src/simd.rs:3417-3578)
runs on the matrix cores; the reference's batch kernels are bit-identical to
its single-token dots (src/simd.rs:8540-8608), so every output row of every
token must equal the oracle's single-token matvec bit for bit.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.test_gpu_kernels import _blocks, _synth_weight

pytestmark = pytest.mark.gpu


def _batch_ref(t, w, xs, rows, cols):
    return np.stack([O.matvec(t, w, x, rows, cols, threads=8) for x in xs])


@pytest.mark.parametrize("t,rows,cols,T", [
    (12, 4096, 4096, 70),    # ragged token tile (K split over a workgroup's waves)
    (12, 4096, 1024, 250),   # a grid of 256 row tiles: one row tile per wave, ragged tokens
    (12, 33, 512, 1),        # one token, partial row tile
    (12, 1000, 256, 64),     # one block per row, exact token tile
    (14, 1024, 14336, 5),    # Q6_K down-projection width
    (14, 300, 5120, 129),    # ragged rows and tokens
])
def test_kquant_batch_bit_exact(hip, t, rows, cols, T):
    w = _synth_weight(t, rows, cols, rows * 3 + cols + T)
    xs = np.random.default_rng(T + cols).standard_normal((T, cols)).astype(np.float32)
    out = np.zeros((T, rows), np.float32)
    assert hip.kquant_matvec_batch_into(t, w, rows, cols, xs, out)
    ref = _batch_ref(t, w, xs, rows, cols)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), np.max(np.abs(out - ref))


@pytest.mark.parametrize("t", [12, 14])
@pytest.mark.parametrize("rows,cols,T", [(96, 1024, 40), (4096, 256, 256)])
def test_kquant_batch_random_blocks(hip, t, rows, cols, T):
    """Uniformly random block bytes: every scale, minimum and quant value the
    formats allow, so the integer sums reach their extremes (Q4_K's largest
    scale digit times the largest nibble included).  The second shape is a
    Q4_K grid large enough for one row tile per wave."""
    rng = np.random.default_rng(t)
    w = _blocks(t, rows * cols // 256, rng)
    xs = (rng.standard_normal((T, cols)) * rng.uniform(0.1, 10, (T, 1))).astype(np.float32)
    xs[3] = 0.0                       # all-zero token: scale 0, quants 0
    xs[5, ::7] = 1e4                  # outliers set the block maxima
    out = np.zeros((T, rows), np.float32)
    assert hip.kquant_matvec_batch_into(t, w, rows, cols, xs, out)
    ref = _batch_ref(t, w, xs, rows, cols)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_kquant_batch_reference_fixture_rows(hip):
    """The reference's own deterministic weights (make_q4k/q6k test builders)
    with its test activation, batched with copies scaled per token."""
    x = O.test_activation(512)
    xs = np.stack([x * s for s in (1.0, -0.5, 3.0)]).astype(np.float32)
    for t, make, seeds in ((12, lambda s: O.make_q4k_weights(4, 512, s, dmin=True), (3, 19)),
                           (14, lambda s: O.make_q6k_weights(4, 512, s), (7, 23))):
        for seed in seeds:
            w = make(seed)
            out = np.zeros((3, 4), np.float32)
            assert hip.kquant_matvec_batch_into(t, w, 4, 512, xs, out)
            assert np.array_equal(out, _batch_ref(t, w, xs, 4, 512))


def test_kquant_batch_rejects_bad_shapes(hip):
    w = _synth_weight(12, 8, 512, 1)
    out = np.zeros((2, 8), np.float32)
    assert not hip.kquant_matvec_batch_into(12, w, 8, 512, np.zeros(1000, np.float32), out)  # not whole rows
    assert not hip.kquant_matvec_batch_into(8, w, 8, 512, np.zeros(1024, np.float32), out)   # not a K-quant
    assert not hip.kquant_matvec_batch_into(12, w, 8, 512, np.zeros(1536, np.float32), out)  # out too small


# ---- resident batched prefill (forward_prefill_batch, src/model.rs:9917-10090) ----
def _pair(name, storage, seed=11):
    from rustyllm_amd import hip, synth
    model = synth.make_model(name, seed=seed)
    return model, hip.Resident(model, storage), O.OracleModel(model, storage, threads=16)


@pytest.fixture
def exact(hip):
    prev = hip.attention_mode("exact")
    yield
    hip.attention_mode(prev)


def _embed(model, tok):
    emb, emb_t = model["token_embd"]
    dim = model["config"]["dim"]
    return O.dequant_row(emb_t, emb[int(tok) * O.row_bytes(emb_t, dim):], dim)


def _assert_kv_equal(model, res, orc, storage, n):
    for layer in range(model["config"]["n_layers"]):
        ok, ov = orc.kv(layer, storage)
        for which, ref in ((0, ok), (1, ov)):
            got = res.kv_read(layer, which, 0, n)
            assert np.array_equal(got.view(np.uint32), ref[:got.size].view(np.uint32)), (layer, which)


@pytest.mark.parametrize("name,n", [("tiny-q4km", 45), ("tiny-qwen", 37), ("tiny-q4km", 300)])
def test_prefill_kv_and_next_logits_bit_exact(hip, exact, name, n):
    """The reference checks batched against sequential prefill to 1e-3
    (src/model.rs:2877-2955); here the cached K/V after prefill and the
    logits of the next decode step equal the oracle's sequential forward bit
    for bit.  n = 300 spans two 256-token chunks."""
    from rustyllm_amd import synth
    storage = 320
    model, res, orc = _pair(name, storage)
    toks = synth.token_ids(5, n + 1, model["config"]["vocab"])
    assert res.prefill(toks[:n], 0)
    for pos in range(n):
        orc.forward(int(toks[pos]), pos, want_logits=False)
    _assert_kv_equal(model, res, orc, storage, n)
    g = res.decode(_embed(model, toks[n]), n, 0, True)
    r = orc.forward(int(toks[n]), n)
    assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), np.max(np.abs(g - r))


def test_prefill_after_decoded_positions(hip, exact):
    """Prefill continuing a cache that decode steps started (start_pos > 0),
    then more decode."""
    from rustyllm_amd import synth
    storage = 128
    model, res, orc = _pair("tiny-q4km", storage, seed=3)
    toks = synth.token_ids(9, 70, model["config"]["vocab"])
    for pos in range(5):
        res.decode(_embed(model, toks[pos]), pos, 0, False)
    assert res.prefill(toks[5:60], 5)
    for pos in range(60):
        orc.forward(int(toks[pos]), pos, want_logits=False)
    for pos in range(60, 70):
        g = res.decode(_embed(model, toks[pos]), pos, 0, True)
        r = orc.forward(int(toks[pos]), pos)
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), pos
    _assert_kv_equal(model, res, orc, storage, 70)


def test_generate_with_batched_prompt_matches_sequential(hip, exact, monkeypatch):
    """generate() prefills all prompt tokens but the last in batches; with
    RUSTY_HIP_PREFILL=0 it decodes them one by one.  Same tokens and logits,
    and both equal the oracle's greedy stream."""
    from rustyllm_amd import synth
    model, res, orc = _pair("tiny-qwen", 200, seed=7)
    prompt = synth.token_ids(31, 90, model["config"]["vocab"])
    a, la = res.generate(prompt, 32, penalty=1.1)
    o, lo = orc.generate(prompt, 32, penalty=1.1)
    assert list(a) == list(o)
    assert np.array_equal(la.view(np.uint32), lo.view(np.uint32))


def test_prefill_refuses_unbatchable_and_bad_ranges(hip):
    """Q8_0 projections are not batchable (standard_prefill_batchable);
    positions past the cache and out-of-range token ids are rejected."""
    from rustyllm_amd import synth
    _, res8, _ = _pair("tiny-q8", 64)
    assert not res8.prefill(np.arange(10), 0)
    model, res, _ = _pair("tiny-q4km", 64)
    assert not res.prefill(np.arange(10), 60)
    assert not res.prefill(np.array([0, model["config"]["vocab"]]), 0)
    assert res.prefill(np.arange(10), 54)
