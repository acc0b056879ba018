"""The division-free scale tables (hephaestus_amd/csrc/scale_tables.h) hold
RN((128+m)/448) and RN(1/that) for every 7-bit mantissa m: compiled with
g++ on the host and compared with runtime IEEE division."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SRC = r'''
#include "scale_tables.h"
#include <cstdio>
int main() {
    volatile float d = 448.0f, one = 1.0f;
    int bad = 0;
    for (int m = 0; m < 128; ++m) {
        float s = (float)(128 + m) / d;
        float inv = one / s;
        if (heph::kScaleTables.scale[m] != s || heph::kScaleTables.inv[m] != inv) ++bad;
    }
    std::printf("%d\n", bad);
    return bad != 0;
}
'''


def test_scale_tables_match_ieee_division(tmp_path):
    src = tmp_path / "t.cpp"
    src.write_text(SRC)
    exe = tmp_path / "t"
    r = subprocess.run(["g++", "-std=c++17", "-O0", "-I",
                        os.path.join(ROOT, "hephaestus_amd", "csrc"), str(src), "-o", str(exe)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        pytest.fail(r.stderr)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "0"
