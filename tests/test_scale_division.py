"""CPU check of the group-scale division in the loop quantizer
(quant_scale_fma in dq8_kernels.hip): for every float m in [2^-100, FLT_MAX],
q0 = m * c with c = 1/127 rounded, r = fma(-q0, 127, m) and fma(r, c, q0)
equal the IEEE quotient m / 127 (weights.rs:117-136, the scale absmax / 127).
The check runs all 1.9e9 values in C with hardware FMA; a planted fault (the
uncorrected q0) must fail it."""
import os
import shutil
import subprocess

import pytest

SOURCE = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
int main(void) {
  const float c = 1.0f / 127.0f;
  unsigned long n = 0, bad = 0;
#pragma omp parallel for reduction(+ : n, bad) schedule(static)
  for (long bl = 0x0D800000L; bl <= 0x7F7FFFFFL; ++bl) {
    const uint32_t b = (uint32_t)bl;
    float m;
    memcpy(&m, &b, 4);
    const float want = m / 127.0f;
    const float q0 = m * c;
    const float r = fmaf(-q0, 127.0f, m);
    const float got = CORRECTED ? fmaf(r, c, q0) : q0 + 0.0f * r;
    uint32_t wb, gb;
    memcpy(&wb, &want, 4);
    memcpy(&gb, &got, 4);
    bad += wb != gb;
    ++n;
  }
  printf("%lu %lu\n", n, bad);
  return 0;
}
"""


def has_fma():
    try:
        with open("/proc/cpuinfo") as f:
            return " fma " in f.read()
    except OSError:
        return False


@pytest.mark.skipif(shutil.which("gcc") is None or not has_fma(), reason="needs gcc and a CPU with FMA")
def test_fma_corrected_quotient_by_127_is_the_ieee_quotient(tmp_path):
    src = tmp_path / "sd.c"
    src.write_text(SOURCE)
    counts = {}
    for corrected in (1, 0):
        exe = tmp_path / f"sd{corrected}"
        subprocess.run(["gcc", "-O2", "-mfma", "-fopenmp", "-ffp-contract=off", f"-DCORRECTED={corrected}",
                        str(src), "-o", str(exe), "-lm"], check=True)
        out = subprocess.run([str(exe)], check=True, capture_output=True, text=True,
                             env=dict(os.environ, OMP_NUM_THREADS="8")).stdout.split()
        counts[corrected] = (int(out[0]), int(out[1]))
    assert counts[1] == (0x7F7FFFFF - 0x0D800000 + 1, 0)
    assert counts[0][1] > 0  # the planted fault is seen
