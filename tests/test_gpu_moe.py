"""GPU parity of the routed MoE block of gpt-oss decode (forward_gpt_oss_into,
src/model.rs:6846-6898) through rusty_hip_moe_ffn, against the oracle's
composition of the reference steps: router matvec + bias, top-k in total
order with the earlier index first among ties and softmax over the chosen
(select_top_logits_into / softmax_selected_into), expert matvecs (MXFP4 in
dot_mxfp4_f32_scalar's order), swiglu_gpt_oss with biases, and the weighted
sum in slot order.  Bit-exact.
"""
import numpy as np
import pytest

from oracle import oracle as O
from rustyllm_amd import synth

pytestmark = pytest.mark.gpu


def _oracle_moe(x, router, rdt, rbias, experts, edt, hidden, biases, k):
    dim = x.size
    n_exp = router.nbytes // O.row_bytes(rdt, dim)
    logits = O.matvec(rdt, router, x, n_exp, dim)
    if rbias is not None:
        logits = (logits + rbias).astype(np.float32)
    idx, _, probs = O.top_k_router(logits, k)
    gate, up, down = experts
    gb, ub, db = biases if biases is not None else (None, None, None)
    rg, rd = O.row_bytes(edt, dim) * hidden, O.row_bytes(edt, hidden) * dim
    moe = np.zeros(dim, np.float32)
    for s, e in enumerate(idx):
        g = O.matvec(edt, gate[e * rg:(e + 1) * rg], x, hidden, dim)
        u = O.matvec(edt, up[e * rg:(e + 1) * rg], x, hidden, dim)
        if gb is not None:
            g = (g + gb[e]).astype(np.float32)
        if ub is not None:
            u = (u + ub[e]).astype(np.float32)
        h = np.array([O.lib.orc_swiglu_gpt_oss(float(a), float(b)) for a, b in zip(g, u)], np.float32)
        d = O.matvec(edt, down[e * rd:(e + 1) * rd], h, dim, hidden)
        if db is not None:
            d = (d + db[e]).astype(np.float32)
        moe = (moe + d * probs[s]).astype(np.float32)
    return moe, idx, probs


def _experts(edt, n_exp, dim, hidden, seed):
    return (synth.normal_quantized(edt, seed, n_exp * hidden, dim, 0.02),
            synth.normal_quantized(edt, seed + 1, n_exp * hidden, dim, 0.02),
            synth.normal_quantized(edt, seed + 2, n_exp * dim, hidden, 0.02))


@pytest.mark.parametrize("dim,hidden,n_exp,k,with_bias", [
    (2880, 2880, 32, 4, True),   # gpt-oss-20B block shape (config 5)
    (256, 128, 8, 2, False),     # Q8_0 router on the Q8_K integer path (K % 256 == 0)
    (96, 160, 5, 3, True),       # ragged: partial row tiles everywhere
])
def test_moe_block_bit_exact(hip, dim, hidden, n_exp, k, with_bias):
    rng = np.random.default_rng(dim + n_exp)
    x = rng.standard_normal(dim).astype(np.float32)
    router = synth.normal_quantized(8, 7 + dim, n_exp, dim, 0.05)
    rbias = (rng.standard_normal(n_exp) * 0.02).astype(np.float32) if with_bias else None
    experts = _experts(39, n_exp, dim, hidden, 100 + dim)
    biases = None
    if with_bias:
        biases = tuple((rng.standard_normal((n_exp, r)) * 0.02).astype(np.float32) for r in (hidden, hidden, dim))
    got = hip.moe_ffn(x, router, 8, rbias, experts, 39, hidden, biases, k)
    assert got is not None
    ref, ridx, rprob = _oracle_moe(x, router, 8, rbias, experts, 39, hidden, biases, k)
    assert list(got[1]) == list(ridx)
    assert np.array_equal(got[2].view(np.uint32), rprob.view(np.uint32))
    assert np.array_equal(got[0].view(np.uint32), ref.view(np.uint32)), np.max(np.abs(got[0] - ref))


def test_moe_router_tie_keeps_earlier_expert(hip):
    """Two experts with identical router rows tie; the reference keeps the
    earlier index first (strict total_cmp greater, src/model.rs:6672, 6712)."""
    dim, hidden, n_exp, k = 256, 64, 6, 2
    rng = np.random.default_rng(3)
    x = rng.standard_normal(dim).astype(np.float32)
    router = synth.normal_quantized(8, 5, n_exp, dim, 0.05)
    rb = O.row_bytes(8, dim)
    router = router.copy()
    # make experts 1 and 4 share the largest row: scale copies of row 0 up
    best = np.argmax(O.matvec(8, router, x, n_exp, dim))
    router[1 * rb:2 * rb] = router[best * rb:(best + 1) * rb]
    router[4 * rb:5 * rb] = router[best * rb:(best + 1) * rb]
    experts = _experts(39, n_exp, dim, hidden, 9)
    got = hip.moe_ffn(x, router, 8, None, experts, 39, hidden, None, k)
    ref, ridx, rprob = _oracle_moe(x, router, 8, None, experts, 39, hidden, None, k)
    assert list(got[1]) == list(ridx)
    assert 1 in list(got[1])
    assert np.array_equal(got[0].view(np.uint32), ref.view(np.uint32))


def test_moe_rejects_bad_arguments(hip):
    x = np.zeros(64, np.float32)
    router = synth.normal_quantized(8, 1, 4, 64, 0.05)
    experts = _experts(39, 4, 64, 32, 2)
    assert hip.moe_ffn(x, router, 8, None, experts, 39, 32, None, 5) is None   # top_k > n_experts
    assert hip.moe_ffn(x, router, 8, None, experts, 39, 32, None, 9) is None   # top_k > 8
