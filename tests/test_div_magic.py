"""The kernels divide lane indices by hd with a multiplier and a shift that
the host computes (osm::div_magic in orthossm_amd/csrc/osm_kernels.h).  This
compiles a host program against that header and checks the method against
integer division: every divisor up to 4096 with every dividend below 70000,
and dividends next to multiples of the divisor up to 2^31 - 1."""
import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

SRC = r"""
#include <stdio.h>
#include "osm_kernels.h"
static inline unsigned umulhi(unsigned a, unsigned b) { return (unsigned)(((unsigned long long)a * b) >> 32); }
int main() {
  long long checked = 0;
  for (unsigned v = 1; v <= 4096; ++v) {
    unsigned m; int s;
    osm::div_magic(v, &m, &s);
    auto check = [&](unsigned n) {
      const unsigned q = (umulhi(n, m) + n) >> s;
      if (q != n / v) { printf("FAIL v=%u n=%u got %u\n", v, n, q); return false; }
      ++checked;
      return true;
    };
    for (unsigned n = 0; n < 70000; ++n) if (!check(n)) return 1;
    for (unsigned long long k = 1; k * v < 0x80000000ull; k = k * 3 + 1) {
      const unsigned long long b = k * v;
      if (!check((unsigned)(b - 1)) || !check((unsigned)b)) return 1;
      if (b + 1 < 0x80000000ull && !check((unsigned)(b + 1))) return 1;
    }
    if (!check(0x7fffffffu)) return 1;
  }
  printf("ok %lld\n", checked);
  return 0;
}
"""


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not found")
def test_division_by_hd_matches_integer_division():
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "t.cpp")
        exe = os.path.join(d, "t")
        with open(src, "w") as f:
            f.write(SRC)
        subprocess.run([HIPCC, "-O2", "-std=c++17", "-I", os.path.join(ROOT, "orthossm_amd", "csrc"), "-o", exe, src],
                       check=True, capture_output=True)
        r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr
