"""Every reference-named export of include/rusty_hip.h called directly through
the C ABI (the symbols a src/hip.rs would bind in place of src/metal.rs:
123-299), each against the oracle row for row, plus the shapes of BASELINE
configs[1] (the full GEMV sweep: four formats at 4096x4096, 14336x4096,
4096x14336 and 128256x4096) and the error convention: 0 for a null pointer,
a zero dimension, a K-quant width that is not a multiple of 256, or a weight
buffer too short for rows x cols (src/metal.rs:716-720,
metal_backend.m:1231-1233)."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _w(t, rows, cols, seed):
    from rustyllm_amd import synth
    return synth.normal_quantized(t, seed, rows, cols, 0.02)


def _x(cols, seed):
    return np.random.default_rng(seed).standard_normal(cols).astype(np.float32)


def _p(a):
    return a.ctypes.data


SINGLE = {"rusty_hip_q4k_matvec": 12, "rusty_hip_q6k_matvec": 14, "rusty_hip_q8_0_matvec": 8,
          "rusty_hip_mxfp4_matvec": 39}


@pytest.mark.parametrize("name", list(SINGLE))
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)])
def test_single_export_config2_shapes(hip, name, rows, cols):
    t = SINGLE[name]
    w = _w(t, rows, cols, rows + 3 * cols + t)
    x = _x(cols, rows + t)
    out = np.zeros(rows, np.float32)
    fn = getattr(hip.lib, name)
    assert fn(_p(w), w.nbytes, _p(x), rows, cols, _p(out)) == 1
    ref = O.matvec(t, w, x, rows, cols, threads=16)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), np.max(np.abs(out - ref))
    hip.weight_cache_clear()


def test_q8_0_export_f32_width(hip):
    """Q8_0 with K % 256 != 0 takes the f32-activation path (dot_q8_0_f32_avx2)."""
    w, x = _w(8, 513, 2880, 5), _x(2880, 5)
    out = np.zeros(513, np.float32)
    assert hip.lib.rusty_hip_q8_0_matvec(_p(w), w.nbytes, _p(x), 513, 2880, _p(out)) == 1
    assert np.array_equal(out, O.matvec(8, w, x, 513, 2880, threads=16))


FUSED = [("rusty_hip_q4k_matvec2", (12, 12)), ("rusty_hip_q6k_matvec2", (14, 14)),
         ("rusty_hip_mxfp4_matvec2", (39, 39)), ("rusty_hip_q4k_matvec3", (12, 12, 12)),
         ("rusty_hip_q6k_matvec3", (14, 14, 14)), ("rusty_hip_q4k_q4k_q6k_matvec3", (12, 12, 14))]


@pytest.mark.parametrize("name,types", FUSED)
def test_fused_exports(hip, name, types):
    """rusty_metal_*_matvec2/3 (src/metal.rs:147-222): one activation, each
    output equal to its own single matvec."""
    cols = 4096
    rows = [4096, 1024, 1024][:len(types)]
    ws = [_w(t, r, cols, 40 + i) for i, (t, r) in enumerate(zip(types, rows))]
    x = _x(cols, 9)
    outs = [np.zeros(r, np.float32) for r in rows]
    args = []
    for w, r in zip(ws, rows):
        args += [_p(w), w.nbytes, r]
    args += [_p(x), cols] + [_p(o) for o in outs]
    assert getattr(hip.lib, name)(*args) == 1
    for o, w, t, r in zip(outs, ws, types, rows):
        assert np.array_equal(o.view(np.uint32), O.matvec(t, w, x, r, cols, threads=16).view(np.uint32))


def test_error_convention(hip):
    lib = hip.lib
    w, x = _w(12, 64, 512, 1), _x(512, 1)
    out = np.zeros(64, np.float32)
    assert lib.rusty_hip_q4k_matvec(_p(w), w.nbytes, _p(x), 64, 512, _p(out)) == 1
    assert lib.rusty_hip_q4k_matvec(None, w.nbytes, _p(x), 64, 512, _p(out)) == 0
    assert lib.rusty_hip_q4k_matvec(_p(w), w.nbytes, None, 64, 512, _p(out)) == 0
    assert lib.rusty_hip_q4k_matvec(_p(w), w.nbytes, _p(x), 64, 512, None) == 0
    assert lib.rusty_hip_q4k_matvec(_p(w), w.nbytes, _p(x), 0, 512, _p(out)) == 0
    assert lib.rusty_hip_q4k_matvec(_p(w), w.nbytes, _p(x), 64, 0, _p(out)) == 0
    assert lib.rusty_hip_q4k_matvec(_p(w), w.nbytes, _p(x), 64, 500, _p(out)) == 0  # cols % 256
    assert lib.rusty_hip_q4k_matvec(_p(w), w.nbytes - 1, _p(x), 64, 512, _p(out)) == 0  # short buffer
    assert lib.rusty_hip_q6k_matvec(_p(w), w.nbytes, _p(x), 64, 512, _p(out)) == 0  # too short for Q6_K
    q = _x(4 * 128, 2)
    kv = _x(16 * 128, 3)
    o = np.zeros(4 * 128, np.float32)
    ok = lib.rusty_hip_attention(_p(q), q.nbytes, _p(kv), kv.nbytes, _p(kv), kv.nbytes, None, 0, _p(o), o.nbytes,
                                 4, 4, 128, 128, 128, 128, 16, 0, 15, C.c_float(0.088), 0)
    assert ok == 1
    # head_dim > 256, a query buffer too short, an output too short
    assert lib.rusty_hip_attention(_p(q), q.nbytes, _p(kv), kv.nbytes, _p(kv), kv.nbytes, None, 0, _p(o), o.nbytes,
                                   1, 1, 512, 512, 512, 512, 4, 0, 3, C.c_float(0.05), 0) == 0
    assert lib.rusty_hip_attention(_p(q), q.nbytes - 4, _p(kv), kv.nbytes, _p(kv), kv.nbytes, None, 0, _p(o),
                                   o.nbytes, 4, 4, 128, 128, 128, 128, 16, 0, 15, C.c_float(0.088), 0) == 0
    assert lib.rusty_hip_attention(_p(q), q.nbytes, _p(kv), kv.nbytes, _p(kv), kv.nbytes, None, 0, _p(o),
                                   o.nbytes - 4, 4, 4, 128, 128, 128, 128, 16, 0, 15, C.c_float(0.088), 0) == 0
