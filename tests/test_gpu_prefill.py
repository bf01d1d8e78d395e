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
    (12, 4096, 4096, 70),    # ragged token tile
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
def test_kquant_batch_random_blocks(hip, t):
    """Uniformly random block bytes: every scale, minimum and quant value the
    formats allow, so the integer sums reach their extremes."""
    rows, cols, T = 96, 1024, 40
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
