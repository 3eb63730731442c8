"""Host-side checks of the arithmetic identities the gfx950 kernels rely on.

hf::rint_div (ascendnpu-ir_amd/csrc/kernels/hf_ops.h) replaces IEEE a/b by
one Markstein correction of a*r with r = RN(1/b).  This compiles the same
three operations for the host (gcc, FMA from libm, no contraction) and checks
them against IEEE division for every mantissa of b, with random a.
"""
import os
import subprocess
import tempfile

SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
static float fbits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint64_t st = 0x9E3779B97F4A7C15ull;
static uint64_t next(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; }
int main(int argc, char **argv) {
  int per_b = 4; long bad = 0, n = 0;
  for (uint32_t m = 0; m < (1u << 23); ++m) {
    volatile float one = 1.0f;
    const float b = fbits(0x3f800000u | m), r = one / b;
    for (int k = 0; k < per_b; ++k) {
      const uint64_t x = next();
      float a = fbits((uint32_t)(0x30000000u + x % 0x1d000000u));  /* 2^-31 .. 2^27 */
      if (x >> 63) a = -a;
      float q = a * r;
      const float e = fmaf(-q, b, a);
      q = fmaf(e, r, q);
      ++n;
      if (q != a / b) ++bad;
    }
  }
  printf("%ld %ld\n", bad, n);
  return 0;
}
"""


def test_one_step_markstein_quotient_is_ieee_division():
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "m.c"), os.path.join(d, "m")
        open(c, "w").write(SRC)
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-o", exe, c, "-lm"], check=True)
        bad, n = map(int, subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split())
    assert n == 4 << 23
    assert bad == 0
