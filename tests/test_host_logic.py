"""Host-side logic of the kernels that needs no GPU.

* ``FastDiv`` (``csrc/cc1d_fastdiv.hpp``): the row kernels split their work
  item index into (row, segment) and (batch entry, channel) with the
  invariant-divisor method of Granlund and Montgomery instead of integer
  division. Compiled here with g++ and checked against plain ``/`` for every
  divisor below 70,000 (row lengths, segment counts and channel counts of
  every test shape), random divisors up to 2^31 and the edge numerators
  (0, d - 1, d, d + 1, 2^31 - 1).
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parent.parent / "causal-conv1d-mojo_amd" / "csrc"

PROGRAM = r"""
#include "cc1d_fastdiv.hpp"
#include <cstdio>
#include <random>
int main() {
    std::mt19937_64 g(1);
    long bad = 0, checked = 0;
    auto check = [&](uint32_t d, int nrand) {
        const cc1d::FastDiv f(d);
        const uint32_t edges[] = {0u, 1u, d - 1, d, d + 1, 2 * d - 1, 2 * d, 0x7ffffffeu, 0x7fffffffu};
        for (uint32_t n : edges)
            if (n < 0x80000000u) { ++checked; if (f.div(n) != n / d) ++bad; }
        for (int i = 0; i < nrand; ++i) {
            const uint32_t n = (uint32_t)(g() & 0x7fffffffu);
            ++checked;
            if (f.div(n) != n / d) ++bad;
        }
    };
    for (uint32_t d = 1; d < 70000; ++d) check(d, 200);
    for (int i = 0; i < 20000; ++i) check((uint32_t)(g() % 0x80000000u) + 1, 200);
    for (int s = 0; s <= 31; ++s) check(1u << s, 200);
    printf("%ld %ld\n", checked, bad);
    return bad != 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not installed")
def test_fastdiv_matches_integer_division(tmp_path):
    src = tmp_path / "fastdiv.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "fastdiv"
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{CSRC}", str(src), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True)
    checked, bad = map(int, res.stdout.split())
    assert res.returncode == 0 and bad == 0, f"{bad} of {checked} quotients differ"
    assert checked > 10_000_000
