"""The wire codec's row-index division (xgen_amd/csrc/fastdiv.h, the same source text the HIP
kernels compile) against C's integer division, on the host with g++."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

CHECK = r"""
#include <cstdio>
#include <cstdlib>
#include "fastdiv.h"
using namespace xgen;
static uint64_t state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd31() { state ^= state << 13; state ^= state >> 7; state ^= state << 17; return (uint32_t)(state >> 33); }
static long bad = 0, checks = 0;
static void check(uint32_t d, uint32_t n) {
  const FastDiv f = make_fastdiv(d);
  ++checks;
  if (fast_div(n, f) != n / d) { if (bad < 10) printf("d=%u n=%u got %u\n", d, n, fast_div(n, f)); ++bad; }
}
static void divisor(uint32_t d) {
  const uint32_t top = 0x7fffffffu;
  check(d, 0); check(d, top); check(d, top - 1);
  for (uint32_t k = 1; k < 64 && (uint64_t)k * d <= top; ++k) { check(d, k * d - 1); check(d, k * d); }
  const uint64_t last = (uint64_t)top / d * d;
  check(d, (uint32_t)last); if (last) check(d, (uint32_t)(last - 1));
  for (int i = 0; i < 2000; ++i) check(d, rnd31());
}
int main() {
  for (uint32_t d = 1; d <= 4096; ++d) divisor(d);
  for (int b = 1; b < 31; ++b) { divisor(1u << b); divisor((1u << b) - 1); divisor((1u << b) + 1); }
  divisor(0x7fffffffu);
  for (int i = 0; i < 4000; ++i) divisor(1 + rnd31());
  printf("%ld checks, %ld bad\n", checks, bad);
  return bad != 0;
}
"""


def test_fast_division_matches_integer_division(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    src = tmp_path / "check.cpp"
    src.write_text(CHECK)
    exe = tmp_path / "check"
    subprocess.run([gxx, "-O2", "-std=c++17", f"-I{ROOT / 'xgen_amd' / 'csrc'}", str(src), "-o", str(exe)],
                   check=True)
    proc = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout
    assert " 0 bad" in proc.stdout
