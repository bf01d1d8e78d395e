"""GPU parity of each decode-step stage against the CPU oracle, through the
C ABI of librusty_hip.so.

Bars: dequantization, Q8_K quantization and
per-block integer dots bit-exact; GEMV and attention within
1e-4 x row L2 norm.  Every GEMV path (Q4_K, Q6_K, Q8_0 on Q8_K activations,
Q8_0 and MXFP4 on f32 activations) reproduces the reference rows bit for bit
and is asserted so; split-K attention is held to 1e-4 * ||o_h|| per head.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests import npref

pytestmark = pytest.mark.gpu


def _blocks(t, n_blocks, rng):
    bsz = {8: 34, 12: 144, 14: 210, 39: 17}[t]
    raw = rng.integers(0, 256, n_blocks * bsz, dtype=np.uint8).reshape(n_blocks, bsz)
    if t == 8:
        raw[:, 1] &= 0x7B
    elif t == 12:
        raw[:, 1] &= 0x7B
        raw[:, 3] &= 0x7B
    elif t == 14:
        raw[:, 209] &= 0x7B
    else:
        raw[:, 16] = rng.integers(100, 150, n_blocks)
    return raw.reshape(-1)


def _synth_weight(t, rows, cols, seed):
    from rustyllm_amd import synth
    return synth.normal_quantized(t, seed, rows, cols, 0.02)


def test_f16_conversion_exhaustive(hip):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = hip.debug_f16(h)
    ref = npref.f16_to_f32(h)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("n", [256, 4096, 14336])
def test_q8k_bit_exact(hip, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * rng.uniform(0.1, 5)).astype(np.float32)
    x[:256] = O.test_activation(256)
    if n > 512:
        x[256:512] = 0.0
    gq, gd, gb = hip.debug_quantize_q8k(x)
    oq, od, ob = O.quantize_q8k(x)
    assert np.array_equal(gq, oq)
    assert np.array_equal(gd.view(np.uint32), od.view(np.uint32))
    assert np.array_equal(gb, ob)


@pytest.mark.parametrize("t,rows,cols", [(8, 7, 2880), (8, 5, 4096), (12, 6, 4096), (14, 6, 5120), (39, 9, 2880)])
def test_dequant_bit_exact(hip, t, rows, cols):
    rng = np.random.default_rng(rows * cols + t)
    w = _blocks(t, rows * cols // O.BLOCK[t][0], rng)
    got = hip.debug_dequant(t, w, rows, cols)
    ref = O.dequant(t, w, rows, cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


FIXTURES = [
    (12, lambda s: O.make_q4k_weights(4, 512, s, dmin=True), [3, 19, 101, 200]),
    (12, lambda s: O.make_q4k_weights(4, 512, s), [1, 2]),
    (14, lambda s: O.make_q6k_weights(4, 512, s), [7, 23, 99, 211]),
    (8, lambda s: np.concatenate([O.make_q8_0_row_scaled(512, (s + r) & 0xFF) for r in range(4)]), [7, 42, 133, 240]),
]


@pytest.mark.parametrize("t,make,seeds", FIXTURES)
def test_block_ints_reference_fixtures(hip, t, make, seeds):
    x = O.test_activation(512)
    qs, d, bs = O.quantize_q8k(x)
    for s in seeds:
        w = make(s)
        got = hip.debug_block_ints(t, w, 4, 512, x)
        rb = O.row_bytes(t, 512)
        for r in range(4):
            a, b = O.block_ints(t, w[r * rb:(r + 1) * rb], qs, bs, 512)
            if t == 12:
                g = got.reshape(4, -1, 2)[r]
                assert np.array_equal(g[:, 0], a) and np.array_equal(g[:, 1], b)
            else:
                assert np.array_equal(got.reshape(4, -1)[r], a)


@pytest.mark.parametrize("t", [8, 12, 14])
def test_block_ints_random(hip, t):
    rng = np.random.default_rng(t)
    rows, cols = 16, 4096
    w = _blocks(t, rows * cols // O.BLOCK[t][0], rng)
    x = rng.standard_normal(cols).astype(np.float32)
    qs, d, bs = O.quantize_q8k(x)
    got = hip.debug_block_ints(t, w, rows, cols, x)
    rb = O.row_bytes(t, cols)
    for r in range(rows):
        a, b = O.block_ints(t, w[r * rb:(r + 1) * rb], qs, bs, cols)
        if t == 12:
            g = got.reshape(rows, -1, 2)[r]
            assert np.array_equal(g[:, 0], a) and np.array_equal(g[:, 1], b)
        else:
            assert np.array_equal(got.reshape(rows, -1)[r], a)


BIT_EXACT_SHAPES = [(12, 33, 512), (12, 4096, 4096), (12, 1024, 14336), (14, 1024, 4096), (14, 513, 14336),
                    (14, 300, 5120), (12, 300, 13824), (8, 2048, 2048), (8, 256, 5632), (8, 77, 4096),
                    (8, 129, 8192), (8, 300, 14336)]


@pytest.mark.parametrize("t,rows,cols", BIT_EXACT_SHAPES)
def test_gemv_bit_exact(hip, t, rows, cols):
    w = _synth_weight(t, rows, cols, rows * 7 + cols)
    x = np.random.default_rng(cols).standard_normal(cols).astype(np.float32)
    out = np.zeros(rows, np.float32)
    assert hip.matvec_into(t, w, x, rows, cols, out)
    ref = O.matvec(t, w, x, rows, cols, threads=8)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), np.max(np.abs(out - ref))


@pytest.mark.parametrize("t,rows,cols", [(39, 2880, 2880), (39, 513, 4096), (39, 200, 14336), (39, 70, 96),
                                         (8, 4096, 2880),
                                         (8, 201, 2880), (8, 9, 160),
                                         (8, 100, 5152)])  # six 32-block chunks through the three-chunk ring
def test_gemv_f32_paths_bit_exact(hip, t, rows, cols):
    """f32-activation rows (MXFP4 always; Q8_0 when K % 256 != 0) in the
    reference's order: dot_mxfp4_f32_scalar's single running sum and
    dot_q8_0_f32_avx2's eight FMA lanes plus hsum_avx (src/simd.rs:5886-5902,
    6671-6692).  Ragged row counts leave partial tiles."""
    w = _synth_weight(t, rows, cols, rows + cols + t)
    x = np.random.default_rng(rows).standard_normal(cols).astype(np.float32)
    out = np.zeros(rows, np.float32)
    assert hip.matvec_into(t, w, x, rows, cols, out)
    ref = O.matvec(t, w, x, rows, cols, threads=8)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), np.max(np.abs(out - ref))


def test_gemv_reference_fixture_rows(hip):
    x = O.test_activation(512)
    for seed in (3, 19, 101, 200):
        w = O.make_q4k_weights(4, 512, seed, dmin=True)
        out = np.zeros(4, np.float32)
        assert hip.q4k_matvec_into(w, x, 4, 512, out)
        assert np.array_equal(out, O.matvec(12, w, x, 4, 512))
    for seed in (7, 23, 99, 211):
        w = O.make_q6k_weights(4, 512, seed)
        out = np.zeros(4, np.float32)
        assert hip.q6k_matvec_into(w, x, 4, 512, out)
        assert np.array_equal(out, O.matvec(14, w, x, 4, 512))


def test_fused_multi_projection_equals_separate(hip):
    """matvec_q4_k3 / kquant3 results equal separate calls (simd.rs:8063-8455)."""
    cols = 4096
    x = np.random.default_rng(1).standard_normal(cols).astype(np.float32)
    a = _synth_weight(12, 4096, cols, 1)
    b = _synth_weight(12, 1024, cols, 2)
    c = _synth_weight(14, 1024, cols, 3)
    outs = [np.zeros(4096, np.float32), np.zeros(1024, np.float32), np.zeros(1024, np.float32)]
    assert hip.quant_matvec3_into((a, 12, 4096), (b, 12, 1024), (c, 14, 1024), x, cols, outs)
    for o, (w, t, r) in zip(outs, ((a, 12, 4096), (b, 12, 1024), (c, 14, 1024))):
        assert np.array_equal(o, O.matvec(t, w, x, r, cols, threads=8))
    o2 = [np.zeros(4096, np.float32), np.zeros(1024, np.float32)]
    assert hip.quant_matvec2_into((a, 12, 4096), (b, 12, 1024), x, cols, o2)
    assert np.array_equal(o2[0], outs[0]) and np.array_equal(o2[1], outs[1])


def test_ffn_and_post_attention_ffn(hip):
    dim, hid = 1024, 2816
    rng = np.random.default_rng(2)
    gate, up = _synth_weight(12, hid, dim, 11), _synth_weight(12, hid, dim, 12)
    down, wo = _synth_weight(14, dim, hid, 13), _synth_weight(12, dim, dim, 14)
    x = rng.standard_normal(dim).astype(np.float32)
    out = np.zeros(dim, np.float32)
    assert hip.q4k_q4k_q6k_ffn_into(gate, up, down, x, dim, hid, dim, hid, out)
    g = O.matvec(12, gate, x, hid, dim)
    u = O.matvec(12, up, x, hid, dim)
    h = O.silu_mul(g, u)
    ref = O.matvec(14, down, h, dim, hid)
    assert np.array_equal(out, ref)
    # post-attention: x += wo*attn; x += down*(silu(gate*n) * up*n), n = rms(x)*norm
    attn = rng.standard_normal(dim).astype(np.float32)
    norm = rng.uniform(0.5, 1.5, dim).astype(np.float32)
    xr = x.copy()
    assert hip.mistral_post_attention_ffn_into(wo, gate, up, down, xr, dim, attn, dim, norm, 1e-5, hid, dim, hid)
    x1 = x + O.matvec(12, wo, attn, dim, dim)
    n = O.rms_norm(x1, norm, 1e-5)
    h = O.silu_mul(O.matvec(12, gate, n, hid, dim), O.matvec(12, up, n, hid, dim))
    ref2 = x1 + O.matvec(14, down, h, dim, hid)
    # the GPU RMSNorm sums in a different order, so its Q8_K of n may differ by
    # one quantum in a few places; the bound allows that, not a missing term.
    assert np.max(np.abs(xr - ref2)) <= 2e-3 * np.linalg.norm(ref2) / np.sqrt(dim)


ATTN = [  # (n_heads, n_kv, head_dim, ctx)
    (32, 8, 128, 512), (32, 8, 128, 4096), (40, 8, 128, 1000), (32, 4, 64, 300), (64, 8, 64, 700),
    (8, 8, 128, 77), (4, 2, 64, 1), (32, 8, 128, 32768),
]


@pytest.fixture(params=["exact", "fast"])
def attn_mode(request, hip):
    prev = hip.attention_mode(request.param)
    yield request.param
    hip.attention_mode(prev)


@pytest.mark.parametrize("nh,nkv,hd,ctx", ATTN)
def test_attention_vs_oracle(hip, attn_mode, nh, nkv, hd, ctx):
    rng = np.random.default_rng(ctx + nh)
    slots = ctx + 5
    q = rng.standard_normal(nh * hd).astype(np.float32)
    K = rng.standard_normal(slots * nkv * hd).astype(np.float32)
    V = rng.standard_normal(slots * nkv * hd).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    out = np.zeros(nh * hd, np.float32)
    assert hip.attention_into(q, K, V, out, nh, nh // nkv, hd, hd, nkv * hd, nkv * hd, slots, 0, ctx - 1, scale)
    ref = O.attention(q, K, V, nh, nkv, hd, hd, nkv * hd, nkv * hd, slots, 0, ctx - 1, scale)
    if attn_mode == "exact":
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
        return
    o = out.reshape(nh, hd)
    r = ref.reshape(nh, hd)
    err = np.abs(o - r).max(axis=1)
    assert np.all(err <= 1e-4 * np.linalg.norm(r, axis=1) + 1e-7), err.max()


@pytest.mark.parametrize("window,pos,slots", [(128, 300, 128), (128, 50, 128), (16, 40, 16)])
def test_attention_sink_window_ring(hip, attn_mode, window, pos, slots):
    rng = np.random.default_rng(pos)
    nh, nkv, hd = 64, 8, 64
    q = rng.standard_normal(nh * hd).astype(np.float32)
    K = rng.standard_normal(slots * nkv * hd).astype(np.float32)
    V = rng.standard_normal(slots * nkv * hd).astype(np.float32)
    sinks = (rng.standard_normal(nh) * 2).astype(np.float32)
    scale = np.float32(0.125)
    for start in (O.lib.orc_attention_start_pos(pos, window), 0):  # windowed and full (ring revisit)
        out = np.zeros(nh * hd, np.float32)
        assert hip.attention_with_sink_into(q, K, V, sinks, out, nh, nh // nkv, hd, hd, nkv * hd, nkv * hd, slots,
                                            start, pos, scale)
        ref = O.attention(q, K, V, nh, nkv, hd, hd, nkv * hd, nkv * hd, slots, start, pos, scale, sinks=sinks)
        if attn_mode == "exact":
            assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
            continue
        r = ref.reshape(nh, hd)
        err = np.abs(out.reshape(nh, hd) - r).max(axis=1)
        assert np.all(err <= 1e-4 * np.linalg.norm(r, axis=1) + 1e-7)


def test_rmsnorm_bit_exact(hip):
    """The sum of squares follows dot_f32_avx2's lane and tree order, so the
    normalised vector matches rms_norm_into bit for bit (incl. tails)."""
    rng = np.random.default_rng(3)
    for n in (2048, 4096, 5120, 2880, 256, 300, 77):
        x = (rng.standard_normal(n) * rng.uniform(0.01, 30)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        got = hip.debug_rmsnorm(x, w, 1e-5)
        ref = O.rms_norm(x, w, 1e-5)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), n


def test_expf_bit_exact(hip):
    """Device expf (restated glibc algorithm) equals the host's libm expf."""
    rng = np.random.default_rng(12)
    x = np.concatenate([
        rng.uniform(-110, 90, 1 << 23).astype(np.float32),
        -np.abs(rng.standard_normal(1 << 22)).astype(np.float32) * 20,
        np.array([0.0, -0.0, 88.0, 88.72283, 88.72284, -103.97, -103.28, -87.3, 1e-30, -1e-30,
                  np.inf, -np.inf, np.nan], np.float32),
        (np.arange(1 << 21, dtype=np.uint32) * 2047).view(np.float32),
    ])
    got = hip.debug_expf(x)
    ref = O.expf(x)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_silu_mul_bit_exact(hip):
    n = 1003 * 8
    gate = ((np.arange(n, dtype=np.float32) / np.float32(n - 1)) * np.float32(180.0) - np.float32(90.0))
    up = (np.sin(np.arange(n, dtype=np.float32) * np.float32(0.37)) * np.float32(2.0)).astype(np.float32)
    got = hip.debug_silu_mul(gate, up)
    ref = O.silu_mul(gate, up, avx2=True)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("neox", [False, True])
def test_rope_bit_exact(hip, neox):
    rng = np.random.default_rng(9)
    hd, nh, nkv = 128, 32, 8
    inv = O.rope_inv_freq(500000.0, hd)
    for pos in (0, 1, 4095, 30000):
        q = rng.standard_normal(nh * hd).astype(np.float32)
        k = rng.standard_normal(nkv * hd).astype(np.float32)
        gq, gk = hip.debug_rope(q, k, pos, hd, nh, nkv, inv, neox=neox)
        rq, rk = O.rope(q, k, pos, hd, nh, nkv, inv, neox=neox)
        assert np.array_equal(gq, rq) and np.array_equal(gk, rk)


def test_greedy_matches_reference(hip):
    rng = np.random.default_rng(4)
    cases = [
        (np.array([8.0, 3.0], np.float32), [0], 4.0),
        (np.array([8.0, 2.5, 2.5], np.float32), [0, 0], 2.0),
        (np.array([np.nan, np.inf, -1.0, -1.0], np.float32), [], 1.0),
        (np.array([np.nan, np.nan], np.float32), [], 1.0),
    ]
    for _ in range(5):
        lg = rng.standard_normal(128256).astype(np.float32)
        lg[rng.integers(0, 128256, 3)] = lg.max()  # exact ties
        rec = list(rng.integers(0, 128256, 64))
        rec[:3] = [int(np.argmax(lg))] * 3
        cases.append((lg, rec, 1.1))
    for lg, rec, pen in cases:
        tok_ref, _ = O.greedy(lg, rec, pen)
        assert hip.debug_greedy(lg, rec, pen) == tok_ref


@pytest.mark.parametrize("t,rows,cols", [(12, 4096, 4096), (14, 1024, 14336), (8, 512, 14336), (39, 300, 4096)])
def test_bench_matvec_equals_oracle_rows(hip, t, rows, cols):
    """The sweep's device-resident GEMV (rusty_hip_bench_matvec, weights
    rotated over device copies) returns the reference rows bit for bit, as
    the per-op export does."""
    w = _synth_weight(t, rows, cols, rows + 3 * cols + t)
    x = np.random.default_rng(cols + t).standard_normal(cols).astype(np.float32)
    got = hip.bench_matvec(t, w, x, rows, cols, 3, 4)
    hip.weight_cache_clear()
    ref = O.matvec(t, w, x, rows, cols, threads=8)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), np.max(np.abs(got - ref))


@pytest.mark.parametrize("ctx", [100, 4096])
def test_bench_attention_exact_and_split_k_agree(hip, ctx):
    """The sweep's attention on device-generated K/V: the exact kernels and
    the split-K kernels (two independent orders of the same softmax) agree
    within 1e-4 x ||o_h|| per head, and both are finite."""
    nh, kvm, hd = 32, 4, 128
    ex = hip.bench_attention(nh, kvm, hd, ctx, 2, 3, 11, "exact").reshape(nh, hd)
    fa = hip.bench_attention(nh, kvm, hd, ctx, 2, 3, 11, "fast").reshape(nh, hd)
    assert np.all(np.isfinite(ex)) and np.all(np.isfinite(fa))
    err = np.abs(ex - fa).max(axis=1)
    assert np.all(err <= 1e-4 * np.linalg.norm(ex, axis=1) + 1e-7), err.max()


def test_mxfp4_gemv_every_scale_byte(hip):
    """MXFP4 rows over random nibbles with every scale byte 0..255 (the
    hardware FP4 conversion for normal scales, the table for the subnormal
    2^-127 and the infinite 2^128), bit-identical to dot_mxfp4_f32_scalar
    (NaN where the reference's arithmetic makes one)."""
    rng = np.random.default_rng(39)
    rows, cols = 256, 2048
    raw = rng.integers(0, 256, (rows, cols // 32, 17), dtype=np.uint8)
    raw[:, :, 16] = (np.arange(rows * (cols // 32)).reshape(rows, -1) * 7) % 256
    w = raw.reshape(-1)
    x = (rng.standard_normal(cols) * 1e-3).astype(np.float32)
    out = np.zeros(rows, np.float32)
    assert hip.matvec_into(39, w, x, rows, cols, out)
    ref = O.matvec(39, w, x, rows, cols, threads=8)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(out[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # rows whose scales avoid 0 and 255 carry finite sums
    assert (~nan).sum() > 0


@pytest.mark.parametrize("rows,cols,scales", [
    (19237, 2880, "normal"),   # > 256 tiles: the one-wave-per-tile kernel; ragged last tile
    (19200, 352, "every"),     # 11 blocks: one partial 16-block chunk; every scale byte
])
def test_mxfp4_gemv_many_tiles(hip, rows, cols, scales):
    """Launches with more 64-row tiles than CUs take the kernel that stages
    16-block chunks through LDS with coalesced loads; its sums stay
    bit-identical to dot_mxfp4_f32_scalar."""
    rng = np.random.default_rng(rows + cols)
    nb = cols // 32
    raw = rng.integers(0, 256, (rows, nb, 17), dtype=np.uint8)
    if scales == "every":
        raw[:, :, 16] = (np.arange(rows * nb).reshape(rows, nb) * 7) % 256
    else:
        raw[:, :, 16] = rng.integers(100, 140, (rows, nb))
    w = raw.reshape(-1)
    x = rng.standard_normal(cols).astype(np.float32)
    out = np.zeros(rows, np.float32)
    assert hip.matvec_into(39, w, x, rows, cols, out)
    ref = O.matvec(39, w, x, rows, cols, threads=8)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(out[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert (~nan).sum() > rows // 2
