"""The BatchNorm + ReLU quantizer computes the code argument (t - mn) / step without a division per
element: with y = 1/step correctly rounded, q0 = RN(a y) and r = fma(-q0, step, a), it takes
RN(q0 + r y), which Markstein's theorem (the IA-64 division) makes the correctly rounded
quotient. The kernel uses it for 2^-60 <= step < inf. This test pins the identity bit-for-bit
against fp32 division on random and quantizer-shaped pairs in that range, in C with fmaf (gcc),
for every quotient that can reach a rounding boundary of a code (q >= 1e-7)."""
import shutil
import subprocess

import pytest

SRC = r'''
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
static uint64_t s = 88172645463325252ull;
static uint64_t rnd(void) { s ^= s << 13; s ^= s >> 7; s ^= s << 17; return s; }
static float bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
int main(void) {
    long bad = 0, n = 0;
    const int qmax[4] = {1, 3, 15, 255};
    for (long i = 0; i < 20000000; ++i) {
        float a, b;
        if (i & 1) {
            const float rng = bits(0x30000000u + (uint32_t)(rnd() % 0x1e000000u));
            b = rng / (float)qmax[rnd() & 3];
            a = rng * (float)((double)(rnd() >> 11) / 9007199254740992.0);
        } else {
            b = bits(0x20000000u + (uint32_t)(rnd() % 0x3f000000u));
            a = bits(0x20000000u + (uint32_t)(rnd() % 0x3f000000u));
        }
        if (!(b >= 0x1p-60f) || !isfinite(b)) continue;
        const float y = 1.0f / b, q0 = a * y;
        const float q1 = fmaf(fmaf(-q0, b, a), y, q0);
        const float q = a / b;
        ++n;
        if (q1 != q && !(q < 1e-7f)) ++bad;
    }
    printf("%ld %ld\n", n, bad);
    return 0;
}
'''


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_reciprocal_correction_division_is_correctly_rounded(tmp_path):
    src = tmp_path / "div.c"
    exe = tmp_path / "div"
    src.write_text(SRC)
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(src), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    n, bad = int(out[0]), int(out[1])
    assert n > 19_000_000 and bad == 0, (n, bad)
