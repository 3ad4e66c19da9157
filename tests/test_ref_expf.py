"""ref_expf (tinyminigo_amd/csrc/kernels/ref_expf.h), the device's expf,
against the C library's expf, which the reference's f32::exp calls (softmax,
src/tensor.rs:1055-1060): bit-identical results.  The header is compiled for
the host with g++ and run over every 61st float bit pattern (70 million
values: all signs, binades, subnormals, infinities and NaNs) plus the
boundary values; the full 2^32 sweep is the same program with stride 1."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "tinyminigo_amd", "csrc", "kernels", "ref_expf.h")

PROGRAM = r"""
#include <math.h>
#include <stdio.h>
#include <string.h>
#include <thread>
#include <vector>
#include <atomic>
#include "ref_expf.h"
static bool same(float a, float b) {
    if (a != a && b != b) return true;
    return memcmp(&a, &b, 4) == 0;
}
int main(int argc, char **argv) {
    const unsigned long long stride = strtoull(argv[1], 0, 10);
    std::atomic<unsigned long long> bad{0}, n{0};
    std::vector<std::thread> th;
    const int NT = 8;
    for (int t = 0; t < NT; t++) th.emplace_back([&, t] {
        unsigned long long b = 0, c = 0;
        for (unsigned long long u = (unsigned long long)t * stride; u < (1ull << 32); u += NT * stride) {
            unsigned ux = (unsigned)u; float x; memcpy(&x, &ux, 4);
            float g = expf(x), m = tmg::ref_expf(x);
            c++;
            if (!same(g, m)) { if (b < 3) printf("x=%a libc=%a ref_expf=%a\n", x, g, m); b++; }
        }
        bad += b; n += c; });
    for (auto &x : th) x.join();
    const float edge[] = {0.0f, -0.0f, 88.0f, -88.0f, 0x1.62e42ep6f, 0x1.62e430p6f, -0x1.9fe368p6f, -0x1.9fe36ap6f,
                          -0x1.9d1d9ep6f, 1e-30f, -1e-30f, 0x1p-149f, __builtin_inff(), -__builtin_inff()};
    for (float x : edge) if (!same(expf(x), tmg::ref_expf(x))) { printf("edge x=%a\n", x); bad++; }
    printf("checked %llu, mismatches %llu\n", n.load(), bad.load());
    return bad.load() != 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_ref_expf_matches_libc_expf(tmp_path):
    src = tmp_path / "check_expf.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "check_expf"
    subprocess.run(["g++", "-O2", "-std=c++17", "-pthread", "-I", os.path.dirname(HEADER), str(src), "-o",
                    str(exe)], check=True)
    r = subprocess.run([str(exe), "61"], capture_output=True, text=True)
    sys.stdout.write(r.stdout)
    assert r.returncode == 0, r.stdout
