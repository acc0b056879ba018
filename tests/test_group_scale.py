"""The division-free group scale (hephaestus_amd/csrc/group_scale.h):
RN(a/7) from an FMA-corrected product and RN(1/q) from one FMA Newton step
must equal IEEE division for every 7-bit mantissa (a = 128 + m), the second
from each of the three f32 values within one ulp of 1/q (the accuracy of
the hardware reciprocal it starts from). Compiled with g++ on the host and
compared with runtime IEEE division; every bf16 amax then runs through the
GPU quantizers in the parity tests."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SRC = r'''
#include "group_scale.h"
#include <cmath>
#include <cstdio>
int main() {
    volatile float seven = 7.0f, d448 = 448.0f, one = 1.0f;
    int bad = 0, checked = 0;
    for (int m = 0; m < 128; ++m) {
        const float a = (float)(128 + m);
        const float q = heph::scale_mant(a);
        if (q != a / seven) ++bad;
        if (q / 64.0f != a / d448) ++bad;              // s mantissa = RN(a/448)
        const float want = one / q;
        const float y0s[3] = {std::nextafter(want, 0.0f), want, std::nextafter(want, 1.0f)};
        for (float y0 : y0s) {
            if (heph::inv_mant(q, y0) != want) ++bad;
            ++checked;
        }
        if (want * 64.0f != one / (q / 64.0f)) ++bad;   // inv mantissa = RN(1/RN(a/448))
    }
    std::printf("%d %d\n", bad, checked);
    return bad != 0;
}
'''


def test_group_scale_matches_ieee_division(tmp_path):
    src = tmp_path / "t.cpp"
    src.write_text(SRC)
    exe = tmp_path / "t"
    r = subprocess.run(["g++", "-std=c++17", "-O2", "-ffp-contract=off", "-I",
                        os.path.join(ROOT, "hephaestus_amd", "csrc"), str(src), "-o", str(exe)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        pytest.fail(r.stderr)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.split() == ["0", "384"], out.stdout


def test_group_scale_catches_a_wrong_formula(tmp_path):
    # the check above must fail for a plain product (no FMA correction)
    src = tmp_path / "t.cpp"
    src.write_text(r'''
#include <cstdio>
int main() {
    volatile float seven = 7.0f, k7 = 1.0f / 7.0f;
    int bad = 0;
    for (int m = 0; m < 128; ++m) { float a = 128 + m; volatile float q = a * k7; if (q != a / seven) ++bad; }
    std::printf("%d\n", bad);
    return 0;
}
''')
    exe = tmp_path / "t"
    subprocess.run(["g++", "-O2", "-ffp-contract=off", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert int(out.stdout) > 0
