"""The multiply-shift divider of the kernels (dq8::Divider, dq8_internal.h).

The wide kernel's tile walk and the quantizer's chunk walk divide by
launch-constant divisors with it: floor(n / d) = (n * mul) >> shift for
0 <= n < 2^31.  This test compiles a host program against the library's own
header and compares every quotient with the integer division: all n below
2^16 for every d up to 4096, and for a spread of divisors up to 2^31 - 1 the
n on both sides of every multiple of d reachable by a sparse walk, up to
2^31 - 1.  A planted fault (mul - 1) must be caught."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "decider-engine_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"

PROGRAM = r"""
#include "dq8_internal.h"
#include <stdio.h>
#include <stdlib.h>
using dq8::Divider;
static int check(uint32_t d, Divider v, uint32_t n) {
  if ((uint32_t)v.div(n) != n / d) {
    printf("mismatch d=%u n=%u got=%d want=%u\n", d, n, v.div(n), n / d);
    return 1;
  }
  return 0;
}
static int run(int planted) {
  const uint32_t top = 0x7fffffffu;
  for (uint32_t d = 1; d <= 4096; ++d) {
    Divider v = Divider::of(d);
    if (planted) v.mul -= 1;
    for (uint32_t n = 0; n < 65536; ++n)
      if (check(d, v, n)) return 1;
    if (check(d, v, top)) return 1;
  }
  uint32_t ds[64];
  int nd = 0;
  for (uint32_t d = 4097; d < top && nd < 40; d = d * 3 + 7) ds[nd++] = d;
  for (int s = 13; s < 31; ++s) ds[nd++] = 1u << s;
  ds[nd++] = top;
  for (int i = 0; i < nd; ++i) {
    const uint32_t d = ds[i];
    Divider v = Divider::of(d);
    if (planted) v.mul -= 1;
    const uint64_t step = (uint64_t)d * ((top / d) / 4096 + 1);
    for (uint64_t m = d; m <= top; m += step)
      for (int e = -1; e <= 1; ++e) {
        const uint64_t n = m + e;
        if (n <= top && check(d, v, (uint32_t)n)) return 1;
      }
    for (int e = 0; e < 3; ++e) {
      const uint64_t m = (uint64_t)(top / d) * d - (uint64_t)e;
      if (check(d, v, (uint32_t)m) || check(d, v, (uint32_t)(m + d - 1 > top ? top : m + d - 1))) return 1;
    }
  }
  return 0;
}
int main(int argc, char** argv) {
  const int planted = argc > 1;
  const int bad = run(planted);
  printf(bad ? "FAIL\n" : "OK\n");
  return 0;
}
"""


@pytest.fixture(scope="module")
def divider_program(tmp_path_factory):
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        pytest.skip("needs hipcc to compile against the HIP headers")
    d = tmp_path_factory.mktemp("divider")
    src, exe = d / "divider_check.cpp", d / "divider_check"
    src.write_text(PROGRAM)
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-I", CSRC, str(src), "-o", str(exe)], check=True,
                   capture_output=True, timeout=300)
    return str(exe)


def test_divider_quotients_are_exact(divider_program):
    out = subprocess.run([divider_program], check=True, capture_output=True, text=True, timeout=300).stdout
    assert out.strip().splitlines()[-1] == "OK", out


def test_divider_check_catches_a_planted_fault(divider_program):
    out = subprocess.run([divider_program, "planted"], check=True, capture_output=True, text=True,
                         timeout=300).stdout
    assert "mismatch" in out and out.strip().splitlines()[-1] == "FAIL", out
