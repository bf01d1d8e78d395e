"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is independent of the oracle's own loops: the reference's test
fixtures and known answers (src/simd.rs, src/model.rs, src/sampling.rs tests),
IEEE/closed forms, vectorized numpy decoders written from the block formats
(tests/npref.py), float64 reductions, and brute-force integer sums.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests import npref


# ---- f16 ---------------------------------------------------------------------------
def test_f16_exhaustive_matches_ieee():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([O.lib.orc_f16_to_f32(int(v)) for v in h], np.float32)
    ref = npref.f16_to_f32(h)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


# ---- MXFP4 scale: mxfp4_scale_lookup_matches_power_formula (simd.rs:7826-7830) --------
@pytest.mark.parametrize("e", [1, 64, 127, 128, 191, 254])
def test_mxfp4_scale_power_of_two(e):
    assert O.lib.orc_mxfp4_scale(e) == np.float32(2.0) ** (e - 127)


def test_mxfp4_scale_extremes():
    assert O.lib.orc_mxfp4_scale(0) == np.ldexp(np.float32(1), -127)
    assert np.isinf(O.lib.orc_mxfp4_scale(255))


# ---- Q8_K quantizer ------------------------------------------------------------------------
@pytest.mark.parametrize("cols", [256, 512, 1024])
def test_q8k_avx2_matches_scalar(cols):
    """q8k_quantizer_simd_matches_scalar (simd.rs:8698-8712)."""
    x = O.test_activation(cols)
    a = O.quantize_q8k(x, avx2=True)
    b = O.quantize_q8k(x, avx2=False)
    for u, v in zip(a, b):
        assert np.array_equal(u, v)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_q8k_closed_form(seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(2048).astype(np.float32) * rng.uniform(0.01, 10)
    x[256:512] = 0.0  # amax == 0 block: d = 0, q = 0
    x[600] = -x[600:856].__abs__().max() * 1.5  # negative extreme sets amax
    qs, d, bs = O.quantize_q8k(x)
    rq, rd, rbs = npref.q8k(x)
    assert np.array_equal(qs, rq)
    assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(bs, rbs)
    assert np.all(qs[256:512] == 0) and d[1] == 0.0


def test_q8k_round_half_even():
    # values landing exactly on .5 after scaling round to even
    x = np.zeros(256, np.float32)
    x[0] = 127.0                       # amax = 127 -> id = 1
    x[1], x[2], x[3], x[4] = 0.5, 1.5, 2.5, -2.5
    qs, d, bs = O.quantize_q8k(x)
    assert list(qs[:5]) == [127, 0, 2, 2, -2]
    assert d[0] == np.float32(127.0) * np.float32(1.0 / 127.0)


# ---- dequantization: bit-exact vs independent decoders -------------------------------------
def _random_blocks(t, n_blocks, rng):
    bsz = {8: 34, 12: 144, 14: 210, 39: 17}[t]
    raw = rng.integers(0, 256, n_blocks * bsz, dtype=np.uint8).reshape(n_blocks, bsz)
    # finite f16 scales (exponent field < 31)
    def fin(col):
        raw[:, col + 1] = raw[:, col + 1] & 0x7B
    if t == 8:
        fin(0)
    elif t == 12:
        fin(0)
        fin(2)
    elif t == 14:
        fin(208)
    elif t == 39:
        raw[:, 16] = rng.integers(100, 150, n_blocks)
    return raw.reshape(-1)


@pytest.mark.parametrize("t,n", [(8, 32 * 37), (12, 256 * 9), (14, 256 * 9), (39, 32 * 45)])
def test_dequant_matches_format_decoder(t, n):
    rng = np.random.default_rng(t)
    w = _random_blocks(t, n // O.BLOCK[t][0], rng)
    got = O.dequant_row(t, w, n)
    ref = npref.DEQ[t](w, n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_tail_zero_filled():
    w = _random_blocks(8, 2, np.random.default_rng(0))
    got = O.dequant_row(8, w, 70)  # 2 whole blocks + 6 tail
    assert np.all(got[64:] == 0.0)


def test_q4k_known_answer_unit_scales():
    """make_q4k_weights (simd.rs:7661-7682): d = 1, dmin = 0 -> w = sc * nibble."""
    w = O.make_q4k_weights(1, 256, 7)
    deq = O.dequant_row(12, w, 256)
    sc, m = npref._k4_scales(w[4:16].reshape(1, 12))
    qs = w[16:144].reshape(4, 32)
    for j in range(4):
        assert np.array_equal(deq[64 * j: 64 * j + 32], (sc[0, 2 * j] * (qs[j] & 0xF)).astype(np.float32))
        assert np.array_equal(deq[64 * j + 32: 64 * j + 64], (sc[0, 2 * j + 1] * (qs[j] >> 4)).astype(np.float32))


# ---- integer dots: int8_parity_test (simd.rs:8890-8925, x86 seeds :8960-9013) --------------
CASES = [
    ("q4k", 12, lambda cols, s: O.make_q4k_weights(1, cols, s, dmin=True), [3, 19, 101, 200]),
    ("q6k", 14, lambda cols, s: O.make_q6k_weights(1, cols, s), [7, 23, 99, 211]),
    ("q8_0", 8, lambda cols, s: O.make_q8_0_row_scaled(cols, s), [7, 42, 133, 240]),
]


@pytest.mark.parametrize("name,t,make,seeds", CASES)
def test_int8_kernel_vs_emulation(name, t, make, seeds):
    cols = 512
    x = O.test_activation(cols)
    qs, d, bs = O.quantize_q8k(x)
    P = O.ptr
    for seed in seeds:
        w = make(cols, seed)
        if t == 12:
            got = O.lib.orc_dot_q4_k_q8k_avx2(P(w), P(qs), P(d), P(bs), cols)
            emu = O.lib.orc_emulate_q4_k_q8k(P(w), P(qs), P(d), P(bs), cols)
            assert got == emu  # same per-block rounding sequence -> identical
        elif t == 14:
            got = O.lib.orc_dot_q6_k_q8k_avx2(P(w), P(qs), P(d), P(bs), cols)
            emu = O.lib.orc_emulate_q6_k_q8k(P(w), P(qs), P(d), cols)
            assert got == emu
        else:
            got = O.lib.orc_dot_q8_0_q8k_avx2(P(w), P(qs), P(d), P(bs), cols)
            emu = O.lib.orc_emulate_q8_0_q8k(P(w), P(qs), P(d), cols)
        assert abs(got - emu) <= 1e-4 * max(abs(emu), 1.0), (seed, got, emu)
        deq = O.dequant_row(t, w, cols)
        reference = float(np.dot(deq.astype(np.float64), x.astype(np.float64)))
        assert abs(got - reference) < 0.10 * abs(reference) + 1.0, (seed, got, reference)


def _bruteforce_q4k(w_row, qs, bs, cols):
    b = w_row.reshape(-1, 144)
    s, m = npref._k4_scales(b[:, 4:16])
    q = b[:, 16:].reshape(-1, 4, 32).astype(np.int64)
    nib = np.stack([q & 0xF, q >> 4], axis=2).reshape(-1, 8, 32)
    x = qs.astype(np.int64).reshape(-1, 8, 32)
    isum = (s.astype(np.int64) * (nib * x).sum(axis=2)).sum(axis=1)
    imin = (m.astype(np.int64) * bs.astype(np.int64).reshape(-1, 8)).sum(axis=1)
    return isum, imin


def _bruteforce_q6k(w_row, qs, cols):
    q, sc, _ = npref.q6_k_ints(w_row, cols)
    x = qs.astype(np.int64).reshape(-1, 256)
    prod = (q.astype(np.int64) * x).reshape(-1, 16, 16).sum(axis=2)
    return (prod * sc.astype(np.int64)).sum(axis=1)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_block_ints_bruteforce(seed):
    rng = np.random.default_rng(seed)
    cols = 1024
    x = rng.standard_normal(cols).astype(np.float32)
    qs, d, bs = O.quantize_q8k(x)
    w4 = _random_blocks(12, cols // 256, rng)
    isum, imin = O.block_ints(12, w4, qs, bs, cols)
    ri, rm = _bruteforce_q4k(w4, qs, bs, cols)
    assert np.array_equal(isum, ri) and np.array_equal(imin, rm)
    w6 = _random_blocks(14, cols // 256, rng)
    isum6, _ = O.block_ints(14, w6, qs, bs, cols)
    assert np.array_equal(isum6, _bruteforce_q6k(w6, qs, cols))
    w8 = _random_blocks(8, cols // 32, rng)
    s8, _ = O.block_ints(8, w8, qs, bs, cols)
    q8 = w8.reshape(-1, 34)[:, 2:].view(np.int8).astype(np.int64)
    assert np.array_equal(s8, (q8 * qs.astype(np.int64).reshape(-1, 32)).sum(axis=1))


@pytest.mark.parametrize("seed", [5, 6])
def test_q4k_row_is_serial_sum_of_block_values(seed):
    """acc += dx * (d*isum - dmin*imin) block by block (simd.rs:6797)."""
    rng = np.random.default_rng(seed)
    cols = 2048
    x = rng.standard_normal(cols).astype(np.float32)
    qs, d, bs = O.quantize_q8k(x)
    w = _random_blocks(12, cols // 256, rng)
    ri, rm = _bruteforce_q4k(w, qs, bs, cols)
    b = w.reshape(-1, 144)
    dd = npref.f16_to_f32(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    dm = npref.f16_to_f32(b[:, 2].astype(np.uint16) | (b[:, 3].astype(np.uint16) << 8))
    acc = np.float32(0.0)
    for i in range(cols // 256):
        acc = np.float32(acc + d[i] * (dd[i] * np.float32(ri[i]) - dm[i] * np.float32(rm[i])))
    got = O.lib.orc_dot_q4_k_q8k_avx2(O.ptr(w), O.ptr(qs), O.ptr(d), O.ptr(bs), cols)
    assert np.float32(got) == acc


# ---- f32-activation dots ---------------------------------------------------------------------
def test_mxfp4_dot_reference_fixture():
    """mxfp4_dot_matches_scalar_reference generator (simd.rs:7836-7858)."""
    blocks = 10
    n = blocks * 32
    row = O.make_mxfp4_test_row(blocks)
    x = O.mxfp4_test_activation(n)
    got = O.lib.orc_dot_mxfp4_f32_scalar(O.ptr(row), O.ptr(x), n)
    ref = float(np.dot(npref.deq_mxfp4(row, n).astype(np.float64), x.astype(np.float64)))
    assert abs(got - ref) <= max(abs(ref), 1.0) * 2e-5


@pytest.mark.parametrize("t,cols", [(8, 2880), (39, 2880), (8, 4096)])
def test_f32_dots_vs_f64(t, cols):
    rng = np.random.default_rng(cols + t)
    w = _random_blocks(t, cols // 32, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    deq = npref.DEQ[t](w, cols).astype(np.float64)
    ref = float(deq @ x.astype(np.float64))
    if t == 8:
        got = O.lib.orc_dot_q8_0_f32_avx2(O.ptr(w), O.ptr(x), cols)
    else:
        got = O.lib.orc_dot_mxfp4_f32_scalar(O.ptr(w), O.ptr(x), cols)
    norm = np.linalg.norm(deq) * np.linalg.norm(x)
    assert abs(got - ref) <= 1e-5 * norm


@pytest.mark.parametrize("rows,threads", [(37, 1), (37, 4), (8, 1), (130, 8)])
def test_mxfp4_matvec_rows_equal_scalar_dot(rows, threads):
    """orc_matvec runs MXFP4 rows eight at a time (independent add chains
    for the CPU); every row must still be dot_mxfp4_f32_scalar's value
    (simd.rs:5886-5902), bit for bit, including the tail rows and every
    scale byte class (normal, subnormal e = 0, infinite e = 255)."""
    rng = np.random.default_rng(rows * 7 + threads)
    cols = 2880
    w = _random_blocks(39, rows * cols // 32, rng)
    w.reshape(-1, 17)[::97, 16] = 0
    w.reshape(-1, 17)[::131, 16] = 255
    x = rng.standard_normal(cols).astype(np.float32)
    y = O.matvec(39, w, x, rows, cols, threads=threads)
    rb = cols // 32 * 17
    for r in range(rows):
        ref = O.lib.orc_dot_mxfp4_f32_scalar(O.ptr(w[r * rb:]), O.ptr(x), cols)
        assert np.float32(ref).view(np.uint32) == y[r].view(np.uint32), r


def test_matvec_dispatch_by_shape():
    """dot_row (simd.rs:962-1060): Q8_0 uses the Q8_K int kernel only when
    cols % 256 == 0, the f32 kernel otherwise."""
    rng = np.random.default_rng(9)
    for cols in (2880, 4096):
        rows = 70
        w = _random_blocks(8, rows * cols // 32, rng)
        x = rng.standard_normal(cols).astype(np.float32)
        y = O.matvec(8, w, x, rows, cols, threads=4)
        rb = O.row_bytes(8, cols)
        qs, d, bs = O.quantize_q8k(x) if cols % 256 == 0 else (None, None, None)
        for r in (0, 33, 69):
            wr = w[r * rb:(r + 1) * rb]
            if cols % 256 == 0:
                e = O.lib.orc_dot_q8_0_q8k_avx2(O.ptr(wr), O.ptr(qs), O.ptr(d), O.ptr(bs), cols)
            else:
                e = O.lib.orc_dot_q8_0_f32_avx2(O.ptr(wr), O.ptr(x), cols)
            assert y[r] == np.float32(e)


def test_matvec_threads_do_not_change_rows():
    rng = np.random.default_rng(11)
    rows, cols = 300, 1024
    w = _random_blocks(12, rows * cols // 256, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    a = O.matvec(12, w, x, rows, cols, threads=1)
    b = O.matvec(12, w, x, rows, cols, threads=8)
    assert np.array_equal(a, b)


# ---- attention --------------------------------------------------------------------------------
def test_attention_start_pos_table():
    """sliding_attention_start_keeps_exact_window_width (model.rs:1535-1546)."""
    f = O.lib.orc_attention_start_pos
    assert [f(0, 2), f(1, 2), f(2, 2), f(3, 2)] == [0, 0, 1, 2]
    assert f(0, 0) == 0 and f(128, 0) == 0


def test_grouped_six_heads_match_individual():
    """grouped_six_head_attention_matches_individual_heads (model.rs:1557-1610)."""
    HD, VD, T = 8, 6, 11
    q = (np.arange(6 * HD, dtype=np.float32) * np.float32(0.013) - np.float32(0.2))
    k = (np.arange(T * HD, dtype=np.float32) * np.float32(0.021) - np.float32(0.3))
    v = (np.arange(T * VD, dtype=np.float32) * np.float32(0.009) - np.float32(0.4))
    scale = np.float32(1.0) / np.sqrt(np.float32(HD))
    grouped = np.zeros(6 * VD, np.float32)
    O.lib.orc_online_attention_grouped(O.ptr(q), O.ptr(k), O.ptr(v), HD, VD, T, HD, VD, 6, 0, T - 1, scale,
                                       O.ptr(grouped))
    for h in range(6):
        e = np.zeros(VD, np.float32)
        qh = np.ascontiguousarray(q[h * HD:(h + 1) * HD])
        O.lib.orc_online_attention(O.ptr(qh), O.ptr(k), O.ptr(v), HD, VD, T, HD, VD, 0, T - 1, scale, O.ptr(e))
        assert np.all(np.abs(grouped[h * VD:(h + 1) * VD] - e) < 1e-5)
    ref = npref.attention_f64(q, k, v, 6, 1, HD, VD, scale)
    assert np.allclose(grouped, ref, atol=1e-6)


def test_ring_slots_match_linearized_window():
    """grouped_attention_ring_slots_match_linearized_window (model.rs:1613-1703)."""
    HD, VD, S, START, END = 8, 6, 5, 7, 11
    q = np.arange(4 * HD, dtype=np.float32) * np.float32(0.017) - np.float32(0.15)
    rk = np.arange(S * HD, dtype=np.float32) * np.float32(0.023) - np.float32(0.31)
    rv = np.arange(S * VD, dtype=np.float32) * np.float32(0.011) - np.float32(0.27)
    order = [2, 3, 4, 0, 1]
    lk = np.concatenate([rk[s * HD:(s + 1) * HD] for s in order])
    lv = np.concatenate([rv[s * VD:(s + 1) * VD] for s in order])
    scale = np.float32(1.0) / np.sqrt(np.float32(HD))
    a = np.zeros(4 * VD, np.float32)
    b = np.zeros(4 * VD, np.float32)
    O.lib.orc_online_attention_grouped(O.ptr(q), O.ptr(rk), O.ptr(rv), HD, VD, S, HD, VD, 4, START, END, scale,
                                       O.ptr(a))
    O.lib.orc_online_attention_grouped(O.ptr(q), O.ptr(lk), O.ptr(lv), HD, VD, S, HD, VD, 4, 0, S - 1, scale,
                                       O.ptr(b))
    assert np.all(np.abs(a - b) < 1e-5)


@pytest.mark.parametrize("nh,nkv,hd,ctx", [(32, 8, 128, 300), (40, 8, 128, 97), (32, 4, 64, 200), (8, 8, 64, 50)])
def test_attention_vs_textbook_f64(nh, nkv, hd, ctx):
    rng = np.random.default_rng(nh + ctx)
    slots = ctx + 7
    q = rng.standard_normal(nh * hd).astype(np.float32)
    K = rng.standard_normal(slots * nkv * hd).astype(np.float32)
    V = rng.standard_normal(slots * nkv * hd).astype(np.float32)
    scale = 1.0 / np.sqrt(hd)
    start, end = 3, ctx - 1
    out = O.attention(q, K, V, nh, nkv, hd, hd, nkv * hd, nkv * hd, slots, start, end, np.float32(scale))
    Kc = K.reshape(slots, -1)[start:end + 1]
    Vc = V.reshape(slots, -1)[start:end + 1]
    ref = npref.attention_f64(q, Kc, Vc, nh, nkv, hd, hd, np.float32(scale))
    assert np.max(np.abs(out - ref)) < 1e-5


def test_sink_attention_vs_textbook_and_window_wrap():
    rng = np.random.default_rng(77)
    nh, nkv, hd, slots = 8, 2, 64, 16
    q = rng.standard_normal(nh * hd).astype(np.float32)
    K = rng.standard_normal(slots * nkv * hd).astype(np.float32)
    V = rng.standard_normal(slots * nkv * hd).astype(np.float32)
    sinks = rng.standard_normal(nh).astype(np.float32) * 2
    pos = 40
    start = O.lib.orc_attention_start_pos(pos, 16)  # 25 .. 40 over a 16-slot ring
    scale = np.float32(0.125)
    out = O.attention(q, K, V, nh, nkv, hd, hd, nkv * hd, nkv * hd, slots, start, pos, scale, sinks=sinks)
    idx = [t % slots for t in range(start, pos + 1)]
    Kc = K.reshape(slots, -1)[idx]
    Vc = V.reshape(slots, -1)[idx]
    ref = npref.attention_f64(q, Kc, Vc, nh, nkv, hd, hd, scale, sinks=sinks)
    assert np.max(np.abs(out - ref)) < 1e-5


def test_full_range_over_ring_revisits_slots():
    """A range longer than the ring walks t % slots repeatedly (model.rs:5783-5786)."""
    rng = np.random.default_rng(3)
    nh, nkv, hd, slots = 4, 1, 64, 8
    q = rng.standard_normal(nh * hd).astype(np.float32)
    K = rng.standard_normal(slots * hd).astype(np.float32)
    V = rng.standard_normal(slots * hd).astype(np.float32)
    out = O.attention(q, K, V, nh, nkv, hd, hd, hd, hd, slots, 0, 19, np.float32(0.1))
    idx = [t % slots for t in range(20)]
    ref = npref.attention_f64(q, K.reshape(slots, -1)[idx], V.reshape(slots, -1)[idx], nh, nkv, hd, hd,
                              np.float32(0.1))
    assert np.max(np.abs(out - ref)) < 1e-5


# ---- small ops -----------------------------------------------------------------------------------
def test_rmsnorm_vs_f64():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(4096).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    out = O.rms_norm(x, w, 1e-5)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean() + 1e-5) * w
    assert np.max(np.abs(out - ref) / (np.abs(ref) + 1e-6)) < 1e-6


@pytest.mark.parametrize("neox", [False, True])
def test_rope_vs_rotation(neox):
    rng = np.random.default_rng(5)
    hd, nh, nkv, pos = 128, 4, 2, 777
    inv = O.rope_inv_freq(500000.0, hd)
    base = 500000.0 ** (np.arange(0, hd, 2) / hd)
    assert np.allclose(inv, 1.0 / base, rtol=1e-6)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    gq, gk = O.rope(q, k, pos, hd, nh, nkv, inv, neox=neox)
    ang = (np.float32(pos) * inv).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    for src, got, n in ((q, gq, nh), (k, gk, nkv)):
        x = src.astype(np.float64).reshape(n, hd)
        if neox:
            a, b = x[:, :hd // 2], x[:, hd // 2:]
            ref = np.concatenate([a * c - b * s, a * s + b * c], axis=1)
        else:
            a, b = x[:, 0::2], x[:, 1::2]
            ref = np.empty_like(x)
            ref[:, 0::2] = a * c - b * s
            ref[:, 1::2] = a * s + b * c
        assert np.max(np.abs(got.reshape(n, hd) - ref)) < 1e-5


def test_rope_gpt_oss_reduces_to_interleaved_and_scales():
    """apply_rope_gpt_oss (model.rs:6603-6636) is apply_rope_qk's adjacent-pair
    rotation with cos and sin scaled by the concentration: at 1.0 it equals
    apply_rope_qk bit for bit, otherwise it is that rotation times c."""
    rng = np.random.default_rng(4)
    hd, nh, nkv = 64, 3, 1
    inv = O.rope_inv_freq(150000.0, hd)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    a_q, a_k = O.rope_gpt_oss(q, k, 37, hd, nh, nkv, 1.0, inv)
    b_q, b_k = O.rope(q, k, 37, hd, nh, nkv, inv)
    assert np.array_equal(a_q, b_q) and np.array_equal(a_k, b_k)
    c = 1.3465736
    s_q, _ = O.rope_gpt_oss(q, k, 37, hd, nh, nkv, c, inv)
    ang = 37.0 * inv.astype(np.float64)
    q2 = q.astype(np.float64).reshape(nh, hd // 2, 2)
    ref = np.stack([q2[..., 0] * np.cos(ang) - q2[..., 1] * np.sin(ang),
                    q2[..., 0] * np.sin(ang) + q2[..., 1] * np.cos(ang)], -1).reshape(-1) * c
    assert np.allclose(s_q, ref, rtol=1e-5, atol=1e-5)


def test_silu_mul_simd_matches_scalar():
    """silu_mul_simd_matches_scalar (simd.rs:9019-9040), incl. the clamp region."""
    n = 1003
    gate = ((np.arange(n, dtype=np.float32) / np.float32(n - 1)) * np.float32(180.0) - np.float32(90.0))
    up = (np.sin(np.arange(n, dtype=np.float32) * np.float32(0.37)) * np.float32(2.0)).astype(np.float32)
    exp = O.silu_mul(gate, up, avx2=False)
    got = O.silu_mul(gate, up, avx2=True)
    tol = np.maximum(1e-5, np.abs(exp) * 1e-5)
    assert np.all(np.abs(got - exp) <= tol)
    g64 = gate.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * up
    assert np.all(np.abs(exp - ref) <= np.maximum(1e-5, np.abs(ref) * 1e-5))


def test_router_topk_matches_full_softmax():
    """Selecting top-k then softmax equals full softmax restricted and
    renormalised (routed MoE test, model.rs:2742-2812); ties keep the earlier
    index (strict total_cmp greater, model.rs:6672)."""
    rng = np.random.default_rng(8)
    for _ in range(20):
        lg = rng.standard_normal(32).astype(np.float32)
        lg[5] = lg[17] = lg.max() + 1  # tie at the top
        idx, val, probs = O.top_k_router(lg, 4)
        order = sorted(range(32), key=lambda i: (-lg[i], i))[:4]
        assert list(idx) == order
        full = np.exp(lg.astype(np.float64) - lg.max())
        sel = full[order] / full[order].sum()
        assert np.allclose(probs, sel, atol=1e-6)


# ---- gpt-oss SwiGLU (model.rs:6596-6600) ----------------------------------------------------------
def _swiglu_f64(g, u):
    g = min(float(g), 7.0) if not np.isnan(g) else 7.0   # f32::min ignores a NaN operand
    u = float(np.clip(u, -7.0, 7.0))                       # clamp keeps NaN
    return g / (1.0 + np.exp(1.702 * -g)) * (u + 1.0)


def test_swiglu_gpt_oss_closed_form_and_clamps():
    f = O.lib.orc_swiglu_gpt_oss
    rng = np.random.default_rng(3)
    for g, u in zip(rng.normal(0, 4, 2000).astype(np.float32), rng.normal(0, 4, 2000).astype(np.float32)):
        ref = _swiglu_f64(g, u)
        assert abs(f(g, u) - ref) <= 4e-7 * max(1.0, abs(ref)), (g, u)
    assert f(0.0, 3.0) == 0.0 and f(2.5, -1.0) == 0.0           # a zero factor
    assert f(100.0, 2.0) == f(7.0, 2.0) and f(1.5, 50.0) == f(1.5, 7.0) and f(1.5, -50.0) == f(1.5, -7.0)
    assert f(float("nan"), 1.0) == f(7.0, 1.0)                    # min(NaN, 7) = 7
    assert np.isnan(f(1.0, float("nan")))
    assert f(-30.0, 0.0) < 0.0 and abs(f(-30.0, 0.0)) < 1e-20     # g * sigmoid(1.702 g) -> -0


# ---- greedy sampling (sampling.rs tests) -------------------------------------------------------------
def test_repeat_penalty_pushes_seen_logits_toward_zero():
    lg = np.array([4.0, -4.0, 2.0], np.float32)
    O.lib.orc_apply_repeat_penalty(O.ptr(lg), 3, O.ptr(np.array([0, 1], np.uint32)), 2, 2.0)
    assert list(lg) == [2.0, -8.0, 2.0]


def test_repeat_penalty_ignores_out_of_range_and_noop():
    lg = np.array([1.0, 2.0], np.float32)
    O.lib.orc_apply_repeat_penalty(O.ptr(lg), 2, O.ptr(np.array([5, 99], np.uint32)), 2, 2.0)
    assert list(lg) == [1.0, 2.0]
    O.lib.orc_apply_repeat_penalty(O.ptr(lg), 2, O.ptr(np.array([0, 1], np.uint32)), 2, 1.0)
    assert list(lg) == [1.0, 2.0]


def test_repeat_penalty_flips_greedy_winner():
    tok, _ = O.greedy(np.array([8.0, 3.0], np.float32), [0], 4.0)
    assert tok == 1


def test_greedy_duplicates_compound_and_first_max_wins():
    tok, lg = O.greedy(np.array([8.0, 2.5, 2.5], np.float32), [0, 0], 2.0)  # 8/2/2 = 2 < 2.5
    assert lg[0] == 2.0 and tok == 1
    tok, _ = O.greedy(np.array([np.nan, np.inf, -1.0, -1.0], np.float32), [], 1.0)
    assert tok == 2
    tok, _ = O.greedy(np.array([np.nan, np.nan], np.float32), [], 1.0)
    assert tok == 0


# ---- bf16 KV cache (KVCache::enable_bf16, model.rs:1406-1421, 6205-6580) ----------
def _bf16_np(x):
    """f32_to_bf16 from the bit layout (round to nearest even, NaN quieted)."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFFFFFF) >> 16
    q = (b >> 16) | 0x40
    return np.where(np.isnan(np.asarray(x, np.float32)), q, r).astype(np.uint16)


def test_f32_to_bf16_closed_form():
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(2000).astype(np.float32),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1.0, -1.5], np.float32),
                        np.array([0x3F808000, 0x3F818000, 0x3F80C000, 0x7F7FFFFF, 0x00000001, 0x7FC00001,
                                  0xFF800001, 0x007FFFFF], np.uint32).view(np.float32)])
    got = O.f32_to_bf16(x)
    assert np.array_equal(got, _bf16_np(x))
    # ties go to even: 1 + 2^-8 exactly between 0x3F80 and 0x3F81 -> 0x3F80; 0x3F818000 -> 0x3F82
    assert got[-8] == 0x3F80 and got[-7] == 0x3F82
    assert got[-5] == 0x7F80  # the largest finite float rounds to +inf
    assert got[-3] & 0x7FC0 == 0x7FC0 and got[-2] & 0xFFC0 == 0xFFC0  # NaNs stay NaN (quiet bit)
    w = np.array([O.lib.orc_bf16_to_f32(int(h)) for h in got[:2000]], np.float32)
    assert np.array_equal(w.view(np.uint32), (got[:2000].astype(np.uint32) << 16))


def test_dot_bf16_single_accumulator_vs_f64():
    rng = np.random.default_rng(6)
    for n in (64, 128, 136, 7):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        got = O.lib.orc_dot_bf16_f32_avx2(O.ptr(a), O.ptr(b), n)
        ref = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        assert abs(got - ref) <= 1e-5 * np.sum(np.abs(a * b)) + 1e-7


def _kv_bf16(rng, slots, w):
    k = rng.standard_normal(slots * w).astype(np.float32)
    v = rng.standard_normal(slots * w).astype(np.float32)
    k16, v16 = _bf16_np(k), _bf16_np(v)
    return k16, v16, (k16.astype(np.uint32) << 16).view(np.float32), (v16.astype(np.uint32) << 16).view(np.float32)


def test_bf16_attention_equals_f32_on_widened_rows_x4():
    """kv_mul 4: dot_bf16x4 / affine_add_bf16x4 are the f32 x4 kernels on the
    widened rows, so bf16 attention over bf16 K/V equals f32 attention over
    the widened values bit for bit (ring ranges included)."""
    rng = np.random.default_rng(7)
    nh, nkv, hd = 8, 2, 128
    slots = 300
    k16, v16, kw, vw = _kv_bf16(rng, slots, nkv * hd)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    for st, en, sl in ((0, 299, 300), (17, 250, 300), (0, 700, 256)):
        got = O.attention_bf16(q, k16, v16, nh, nkv, hd, hd, nkv * hd, nkv * hd, sl, st, en, np.float32(0.088))
        ref = O.attention(q, kw, vw, nh, nkv, hd, hd, nkv * hd, nkv * hd, sl, st, en, np.float32(0.088))
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("nh,nkv", [(4, 4), (10, 2), (16, 2), (12, 2)])
def test_bf16_attention_vs_f64(nh, nkv):
    """Other group sizes (single-accumulator dots for every head) against the
    textbook softmax in float64 over the widened values."""
    rng = np.random.default_rng(nh * 10 + nkv)
    hd, ctx = 64, 333
    k16, v16, kw, vw = _kv_bf16(rng, ctx, nkv * hd)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    scale = np.float32(0.125)
    got = O.attention_bf16(q, k16, v16, nh, nkv, hd, hd, nkv * hd, nkv * hd, ctx, 0, ctx - 1, scale)
    ref = npref.attention_f64(q, kw.reshape(ctx, -1), vw.reshape(ctx, -1), nh, nkv, hd, hd, scale)
    r = ref.reshape(nh, hd)
    assert np.all(np.abs(got.reshape(nh, hd) - r).max(axis=1) <= 1e-5 * np.linalg.norm(r, axis=1) + 1e-6)
