"""CPU-side checks of the product library: it loads, exports every symbol the
header declares, reports unavailable without a GPU, and the host-side
quantizers write blocks that decode back to the source within format error."""
import ctypes
import os
import re

import numpy as np
import pytest

from tests import npref

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_symbols():
    text = open(os.path.join(ROOT, "include", "rusty_hip.h")).read()
    return sorted(set(re.findall(r"\b(rusty_hip_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    from rustyllm_amd import hip
    syms = _header_symbols()
    assert len(syms) >= 30
    for s in syms:
        assert hasattr(hip.lib, s), s
    assert set(hip.SYMBOLS) == set(syms)


def test_unavailable_without_gpu(monkeypatch):
    from rustyllm_amd import hip
    from tests.conftest import gpu_present
    if gpu_present():
        pytest.skip("GPU present")
    assert hip.lib.rusty_hip_available() == 0
    out = np.zeros(4, np.float32)
    assert not hip.q4k_matvec_into(np.zeros(4 * 144, np.uint8), np.zeros(256, np.float32), 4, 256, out)
    monkeypatch.setenv("RUSTY_HIP", "0")
    assert not hip.available()


def test_resident_desc_layout_matches_reference_repr_c():
    """ResidentLayerDesc (src/metal.rs:347-360): 7 pointers, 7 usize, 7 u32,
    7 u32, two pointers, then three (pointer, u32) pairs."""
    from rustyllm_amd import hip
    D = hip.ResidentLayerDesc
    assert D.w.offset == 0 and D.w_len.offset == 56 and D.w_rows.offset == 112 and D.w_dt.offset == 140
    assert D.attn_norm.offset == 168 and D.bq.offset == 184 and D.bv_len.offset == 224
    assert ctypes.sizeof(D) == 232


@pytest.mark.parametrize("t,tol", [(8, 0.01), (12, 0.12), (14, 0.035), (39, 0.25)])
def test_quantizers_round_trip(t, tol):
    from rustyllm_amd import synth
    x = synth.normal_f32(42, 64, 512, 0.02)
    q = synth.quantize(t, x)
    back = npref.DEQ[t](q, x.size).reshape(x.shape)
    rel = np.linalg.norm(back - x) / np.linalg.norm(x)
    assert rel < tol, rel


def test_normal_generator_is_thread_independent_and_gaussian():
    from rustyllm_amd import synth
    a = synth.normal_f32(7, 200, 1000, 0.02)
    b = synth.normal_f32(7, 200, 1000, 0.02)
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 2e-4 and abs(a.std() - 0.02) < 2e-4
    assert not np.array_equal(a, synth.normal_f32(8, 200, 1000, 0.02))


def test_rope_inv_freq_matches_reference_formula():
    from rustyllm_amd import synth
    from oracle import oracle as O
    for theta, hd in ((10000.0, 64), (500000.0, 128), (1000000.0, 128)):
        assert np.array_equal(synth.rope_inv_freq(theta, hd), O.rope_inv_freq(theta, hd))
