"""The kernels divide by launch-invariant integers (positions per block, chunks per row)
with qubivex_amd/csrc/fastdiv.h.  This compiles that header for the host with g++ and
checks it against C's `/` for divisors 1..4096, powers of two and large divisors, on edge
and random numerators over the whole 32-bit range."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
HDR = os.path.join(os.path.dirname(HERE), "qubivex_amd", "csrc")

PROG = r"""
#include "fastdiv.h"
#include <stdio.h>
#include <stdint.h>
static uint64_t st = 0x9e3779b97f4a7c15ull;
static uint32_t rnd(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return (uint32_t)st; }
static int check(uint32_t d) {
    qvkv::FastDiv f(d);
    uint32_t edge[] = {0u, 1u, d - 1u, d, d + 1u, 2u * d - 1u, 0x7fffffffu, 0x80000000u,
                       0xfffffffeu, 0xffffffffu, 0xffffffffu - 0xffffffffu % d,
                       0xffffffffu - 0xffffffffu % d - 1u};
    for (uint32_t n : edge)
        if (f.div(n) != n / d) { printf("FAIL d=%u n=%u\n", d, n); return 1; }
    for (int i = 0; i < 20000; i++) {
        uint32_t n = rnd() >> (rnd() & 31u);
        if (f.div(n) != n / d) { printf("FAIL d=%u n=%u\n", d, n); return 1; }
    }
    return 0;
}
int main() {
    int bad = 0;
    for (uint32_t d = 1; d <= 4096; d++) bad |= check(d);
    for (int s = 0; s < 32; s++) { bad |= check(1u << s); bad |= check((1u << s) + 1u); bad |= check((1u << s) - 1u ? (1u << s) - 1u : 1u); }
    for (int i = 0; i < 2000; i++) { uint32_t d = rnd(); bad |= check(d ? d : 1u); }
    bad |= check(0xffffffffu);
    if (!bad) printf("OK\n");
    return bad;
}
"""


def test_fastdiv_matches_division(tmp_path):
    src = tmp_path / "fd.cpp"
    src.write_text(PROG)
    exe = tmp_path / "fd"
    try:
        subprocess.run(["g++", "-O2", "-std=c++17", "-I", HDR, str(src), "-o", str(exe)],
                       check=True, capture_output=True, text=True)
    except FileNotFoundError:
        pytest.skip("g++ is not available")
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "OK", r.stdout
