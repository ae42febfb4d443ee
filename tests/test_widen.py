"""The integer float -> double widening of the strip engine's float64 window
weights (csrc/fa_widen.h: widen_uniform) against the conversion, for every
one of the 2^32 float bit patterns (built with g++ on the host, ~10 s)."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "frame_analytics_amd" / "csrc"

MAIN = r"""
#include <cstdio>
#include <cstring>
#include "fa_widen.h"
int main() {
  unsigned long long bad = 0;
  for (unsigned long long i = 0; i <= 0xffffffffull; ++i) {
    const uint32_t u = static_cast<uint32_t>(i);
    float f;
    std::memcpy(&f, &u, 4);
    const double a = fa::widen_uniform(f), b = static_cast<double>(f);
    uint64_t x, y;
    std::memcpy(&x, &a, 8);
    std::memcpy(&y, &b, 8);
    if (x != y && bad++ < 4) std::printf("%08x: %016llx != %016llx\n", u,
                                         (unsigned long long)x, (unsigned long long)y);
  }
  std::printf("mismatches %llu\n", bad);
  return bad != 0;
}
"""


def test_widen_uniform_matches_the_conversion(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    src = tmp_path / "widen.cpp"
    src.write_text(MAIN)
    exe = tmp_path / "widen"
    subprocess.run([gxx, "-O2", "-std=c++17", "-D__host__=", "-D__device__=", f"-I{CSRC}",
                    str(src), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout
    assert "mismatches 0" in r.stdout
