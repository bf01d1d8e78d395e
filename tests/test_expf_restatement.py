"""Pins the device expf (rustyllm_amd/csrc/attention_exact.hip, expf_glibc)
on the CPU: the exp2 table equals 2^(i/32) rounded to double (computed here
with exact decimal arithmetic), and a C twin of the device function (same
constants, same fused operations) agrees with this machine's libm expf on a
strided sweep of float inputs.  The reference's exp_attn is f32::exp, i.e.
libm expf (src/model.rs:5720-5726).  The full 2^32 sweep of the same twin
found 0 mismatches against glibc 2.35."""
import os
import re
import struct
import subprocess
import tempfile
from decimal import Decimal, getcontext

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "rustyllm_amd", "csrc", "attention_exact.hip")


def _device_table():
    text = open(SRC).read()
    body = text[text.index("kExp2fTab[32] = {"):]
    body = body[: body.index("};")]
    return [int(v, 16) for v in re.findall(r"0x([0-9a-f]{16})ull", body)]


def test_exp2_table_is_exact():
    getcontext().prec = 80
    tab = _device_table()
    assert len(tab) == 32
    for i, v in enumerate(tab):
        d = float(Decimal(2) ** (Decimal(i) / Decimal(32)))
        bits = struct.unpack("<Q", struct.pack("<d", d))[0]
        assert v == (bits - (i << 47)) & 0xFFFFFFFFFFFFFFFF, i


TWIN = r"""
#include <stdio.h>
#include <stdint.h>
#include <string.h>
#include <math.h>
static const uint64_t TAB[32] = { %s };
static inline uint32_t asu(float f){uint32_t u; memcpy(&u,&f,4); return u;}
static float twin(float x) {
    uint32_t abstop = (asu(x) >> 20) & 0x7ff;
    if (abstop >= (0x42b00000u >> 20)) {
        if (asu(x) == 0xff800000u) return 0.0f;
        if (abstop >= (0x7f800000u >> 20)) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32768.0, c1 = 0x1.ebfce50fac4f3p-3 / 1024.0, c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    double xd = x, kd = fma(inv, xd, shift); uint64_t ki; memcpy(&ki, &kd, 8); kd -= shift;
    double r = fma(inv, xd, -kd); uint64_t t = TAB[ki %% 32] + (ki << 47); double s; memcpy(&s, &t, 8);
    double z = fma(c0, r, c1), r2 = r * r, y = fma(c2, r, 1.0); y = fma(z, r2, y);
    return (float)(y * s);
}
int main(void) {
    long bad = 0, n = 0;
    for (uint64_t u = 0; u < (1ull << 32); u += 61) {
        uint32_t b = (uint32_t)u; float x; memcpy(&x, &b, 4);
        float a = expf(x), m = twin(x); n++;
        if (asu(a) != asu(m) && !(isnan(a) && isnan(m))) bad++;
    }
    printf("%%ld %%ld\n", n, bad);
    return 0;
}
"""


def test_c_twin_matches_libm_expf():
    tab = ", ".join("0x%016xull" % v for v in _device_table())
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "t.c"), os.path.join(d, "t")
        open(src, "w").write(TWIN % tab)
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()
    n, bad = int(out[0]), int(out[1])
    assert n > 70_000_000 and bad == 0
