"""The opt-in matrix-core expert product of the batched gpt-oss prefill
(rusty_hip_set_expert_mfma, rusty_hip_mxfp4_experts with mfma = 1).

The reference sums every MXFP4 row serially (dot_mxfp4_f32_scalar,
src/simd.rs:5886-5902); the matrix cores add the same f32 products in their
own order.  The weights lut[n] * 2^(e-127) are exact in f32 either way, so
each product may differ from the serial sum by rounding only: it is held to
1e-4 * sum_k |w_k x_k| per (pair, row).  The serial path (mfma = 0, the
default) is checked bit for bit against the oracle's matvec on the same
inputs, so both paths are anchored on the reference's arithmetic.
"""
import numpy as np
import pytest

from oracle import oracle as O
from rustyllm_amd import synth

pytestmark = pytest.mark.gpu

MX = 39


def _experts(n_exp, rows, cols, seed, dequant=True):
    """Expert matrices with rows padded to a 16-byte stride; a few blocks get
    the subnormal scale byte 0 (the table path of the decode)."""
    rb = synth.row_bytes(MX, cols)
    stride = (rb + 15) // 16 * 16
    w = np.zeros((n_exp, rows, stride), np.uint8)
    rng = np.random.default_rng(seed)
    for e in range(n_exp):
        q = synth.normal_quantized(MX, seed + 7 * e, rows, cols, std=0.05).reshape(rows, rb)
        w[e, :, :rb] = q
        for _ in range(3):
            r, b = int(rng.integers(rows)), int(rng.integers(cols // 32))
            w[e, r, 17 * b + 16] = 0  # scale byte of block b
    if not dequant:
        return w, stride, None
    deq = np.stack([O.dequant(MX, np.ascontiguousarray(w[e, :, :rb]), rows, cols) for e in range(n_exp)])
    return w, stride, deq


def _routing(T, k, n_exp, seed, unused=()):
    rng = np.random.default_rng(seed)
    pool = [e for e in range(n_exp) if e not in unused]
    sel = np.stack([rng.choice(pool, size=k, replace=False) for _ in range(T)]).astype(np.int32).reshape(-1)
    return sel


@pytest.mark.parametrize("x_per_pair,shape", [
    (False, (6, 300, 2880, 70, 3)),     # ragged row tile, an empty expert, several pair tiles
    (True, (6, 300, 2880, 70, 3)),
    (False, (32, 2880, 2880, 256, 4)),  # a gpt-oss-20B gate/up launch (1024 pairs)
    (True, (32, 2880, 2880, 256, 4)),   # ... and its down launch
])
def test_expert_product_mfma_within_tolerance(hip, x_per_pair, shape):
    import torch
    dev = torch.device("cuda:0")
    n_exp, rows, cols, T, k = shape
    w, stride, _ = _experts(n_exp, rows, cols, 41, dequant=False)
    sel = _routing(T, k, n_exp, 5, unused=(4,))
    n_pairs = T * k
    counts = np.bincount(sel, minlength=n_exp)
    assert counts[4] == 0 and counts.max() > 32  # an empty expert and one of several 32-pair tiles
    nx = n_pairs if x_per_pair else T
    x = synth.normal_f32(9, nx, cols)
    tw, tx, ts = (torch.from_numpy(a).to(dev) for a in (w.reshape(-1), x.reshape(-1), sel))
    ldy = rows + 4
    outs = []
    for mfma in (0, 1):
        ty = torch.full((n_pairs * ldy,), float("nan"), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        assert hip.mxfp4_experts_dev(tw.data_ptr(), stride, rows * stride, n_exp, rows, cols, tx.data_ptr(), cols,
                                     x_per_pair, k, ts.data_ptr(), n_pairs, ty.data_ptr(), ldy, mfma)
        outs.append(ty.cpu().numpy().reshape(n_pairs, ldy)[:, :rows])
    exact, fast = outs
    rb = synth.row_bytes(MX, cols)
    worst = 0.0
    # the serial path against the oracle (every pair of the small shape, every
    # 37th at the 20B shape), the matrix cores against the bound for all
    check = set(range(0, n_pairs, 1 if n_pairs < 1000 else 37))
    for e in range(n_exp):
        ps = np.nonzero(sel == e)[0]
        if ps.size == 0:
            continue
        we = np.ascontiguousarray(w[e, :, :rb])
        deq = O.dequant(MX, we, rows, cols)
        xs = x[ps] if x_per_pair else x[ps // k]
        bound = 1e-4 * (np.abs(xs) @ np.abs(deq).T) + 1e-30
        err = np.abs(fast[ps] - exact[ps])
        assert np.all(err <= bound), (e, float(np.max(err / bound)))
        worst = max(worst, float(np.max(err / bound)))
        for i, p in enumerate(ps):
            if p in check:
                ref = O.matvec(MX, we, xs[i], rows, cols)
                assert np.array_equal(exact[p].view(np.uint32), ref.view(np.uint32)), p
    print(f"expert mfma {shape}: worst |error| / (1e-4 sum|w x|) = {worst:.3g}")


def test_expert_product_rejects_bad_arguments(hip):
    import torch
    dev = torch.device("cuda:0")
    tw = torch.zeros(4 * 64 * 96, dtype=torch.uint8, device=dev)
    tx = torch.zeros(64 * 96, dtype=torch.float32, device=dev)
    ts = torch.zeros(64, dtype=torch.int32, device=dev)
    ty = torch.zeros(64 * 64, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    ok = dict(w_ptr=tw.data_ptr(), row_stride=64, exp_stride=64 * 64, n_exp=4, rows=64, cols=96,
              x_ptr=tx.data_ptr(), ldx=96, x_per_pair=False, top_k=1, sel_ptr=ts.data_ptr(), n_pairs=64,
              y_ptr=ty.data_ptr(), ldy=64, mfma=True)
    assert hip.mxfp4_experts_dev(**ok)
    for bad in (dict(cols=80), dict(row_stride=60), dict(row_stride=48), dict(n_exp=65), dict(top_k=9),
                dict(n_pairs=1025), dict(ldy=63), dict(exp_stride=64 * 63)):
        assert not hip.mxfp4_experts_dev(**{**ok, **bad}), bad


@pytest.mark.parametrize("name,max_len,pieces", [
    ("tiny-gptoss", 80, [(0, 30), (30, 61)]),
    ("tiny-gptoss-w128", 512, [(0, 200), (200, 390)]),
])
def test_gptoss_prefill_with_expert_mfma(hip, name, max_len, pieces):
    """The batched gpt-oss prefill with the matrix-core expert product: the
    first layer's K/V (before any expert product) stay bit-exact, every later
    layer's K/V and the next step's logits are within a relative 1e-3 of the
    oracle's sequential forward, and the greedy stream after the prompt is
    compared with the exact prefill's (the number of identical tokens is
    printed)."""
    prev_mode = hip.attention_mode("exact")
    prev = hip.set_expert_mfma(True)
    try:
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
            for which, ref in ((0, orc.kc[layer]), (1, orc.vc[layer])):
                got = res.kv_read(layer, which, 0, S)
                if layer == 0:
                    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
                else:
                    assert np.max(np.abs(got - ref)) <= 1e-3 * np.max(np.abs(ref)), (layer, which)
        emb, et = model["token_embd"]
        x = O.dequant_row(et, emb[int(toks[n]) * O.row_bytes(et, cfg["dim"]):], cfg["dim"])
        g = res.decode(x, n, 0, True)
        r = orc.forward(int(toks[n]), n)
        rel = float(np.max(np.abs(g - r)) / np.max(np.abs(r)))
        assert rel <= 1e-3, rel
        # greedy continuation after a batched prompt: matrix cores against exact
        prompt = synth.token_ids(4, n, cfg["vocab"])
        a_toks, _ = hip.ResidentGptOss(model, max_len).generate(prompt, 16, penalty=1.1)
        hip.set_expert_mfma(False)
        b_toks, _ = hip.ResidentGptOss(model, max_len).generate(prompt, 16, penalty=1.1)
        same = int(np.sum(np.asarray(a_toks) == np.asarray(b_toks)))
        print(f"{name}: next-logit relative error {rel:.3g}; greedy tokens equal to the exact prefill's: {same}/16")
    finally:
        hip.set_expert_mfma(prev)
        hip.attention_mode(prev_mode)
