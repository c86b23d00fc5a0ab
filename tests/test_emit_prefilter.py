"""Pin of the emit scan's prefilter (k_i8_emit in fanarvse_paper_amd/csrc/fvs_scan.hip).

The kernel tests every (query, row) element with
    g = fmaf((float)acc, z, z + z) >= T,   T = (t0 - qcp)/qs - 2^-20 (|t0| + |qcp|)/qs
and computes the canonical estimate est = fmaf((float)acc * qs, z, qcp) only for elements that pass g;
the emitted set is {est >= t0}. That is exact only if no element with est >= t0 fails g. This test
checks that claim by brute force in IEEE f32 (a C program built with -ffp-contract=off, whose fmaf is
the correctly rounded fused multiply-add, like v_fma_f32): random scales, centre terms and accumulators
over the whole int8 range, thresholds placed on and next to an element's own estimate, and every
accumulator within 40 of it. A planted mistake (the margin added to T instead of subtracted) must
produce misses, so the check can fail.
"""
import shutil
import subprocess

import pytest

SRC = r"""
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
static int planted = 0;
static float prefilter_T(float th, float qc, float qsv) {  /* emit_prefilter_T */
  if (!(qsv > 0.f)) return -INFINITY;
  const float b = (th - qc) / qsv;
  const float m = (fabsf(th) + fabsf(qc)) * (0x1p-20f / qsv);
  const float T = planted ? b + m : b - m;
  if (!(T < INFINITY)) return th == INFINITY ? INFINITY : -INFINITY;
  return T;
}
static unsigned long long s = 88172645463325252ull;
static double rnd(void) { s ^= s << 13; s ^= s >> 7; s ^= s << 17; return (s >> 11) * (1.0 / 9007199254740992.0); }
int main(int argc, char **argv) {
  planted = argc > 1;
  long miss = 0, pass = 0;
  for (int it = 0; it < 300000; it++) {
    const float qs = (float)pow(10, -6 + 5 * rnd());
    float z = (float)pow(10, -7 + 5 * rnd());
    if (it % 97 == 0) z = (float)(1e-14 * (1 + rnd()));
    const float qcp = (float)(2 * rnd() - 1) * (it % 5 == 0 ? 100.f : 1.f);
    const int a0 = (int)((2 * rnd() - 1) * 4194304);
    const float e0 = fmaf((float)a0 * qs, z, qcp);
    float t0 = nextafterf(e0, (it & 1) ? INFINITY : -INFINITY);
    if (it % 3 == 0) t0 = e0;
    const float T = prefilter_T(t0, qcp, qs);
    const float add = z + z;
    for (int d = -40; d <= 40; d++) {
      const int acc = a0 + d;
      if (acc > 4194304 || acc < -4194304) continue;
      const int exact = fmaf((float)acc * qs, z, qcp) >= t0;
      const int g = fmaf((float)acc, z, add) >= T;
      pass += exact;
      if (exact && !g) miss++;
    }
  }
  printf("%ld %ld\n", pass, miss);
  return 0;
}
"""


def _run(tmp_path, planted):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "prefilter.c"
    exe = tmp_path / "prefilter"
    src.write_text(SRC)
    subprocess.run([cc, "-O2", "-ffp-contract=off", "-o", str(exe), str(src), "-lm"], check=True)
    out = subprocess.run([str(exe)] + (["planted"] if planted else []), check=True, capture_output=True, text=True)
    passed, missed = (int(x) for x in out.stdout.split())
    return passed, missed


def test_prefilter_never_drops_a_passing_element(tmp_path):
    passed, missed = _run(tmp_path, planted=False)
    assert passed > 1_000_000
    assert missed == 0


def test_prefilter_check_catches_a_wrong_margin_sign(tmp_path):
    _, missed = _run(tmp_path, planted=True)
    assert missed > 0
