"""The quotient the fp8 quantisers use in place of the IEEE division (csrc/common.h div_rn):
q = a * rb, rb = 1/b; result = copysign(fma(fma(-q, b, a), rb, q), a), for b in [2^-64, 2^100].

Checked here on the host, where the same four operations are the C library's correctly rounded
float arithmetic: against a / b bit for bit for |a| >= 2^-100 (and a == 0, both signs), and through
the e4m3 encoding (RNE, saturating at 448) for every a -- signed zeros, subnormals, values beside
the e4m3 rounding midpoints of the quotient, the scale range's edges.  The device kernels are
checked against the oracle on such inputs in test_gpu_fp8_quant_edges.py."""
from __future__ import annotations

import shutil
import subprocess
import textwrap

import pytest

_SRC = textwrap.dedent(r"""
    #include <math.h>
    #include <stdint.h>
    #include <stdio.h>
    #include <stdlib.h>
    #include <string.h>
    static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
    static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
    static uint64_t st = 0x2545F4914F6CDD1Dull;
    static uint64_t xr(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; }
    static uint8_t e4m3(float f) {  /* OCP e4m3fn, RNE, saturating at 448 */
      uint32_t u = f2u(f); uint8_t sign = (u >> 24) & 0x80; uint32_t a = u & 0x7fffffff;
      if (a > 0x7f800000u) return sign | 0x7f;
      if (a >= 0x43e00000u) return sign | 0x7e;
      if (a < 0x3c800000u) return sign | (uint8_t)rintf(u2f(a) * 512.0f);
      uint32_t keep = (a & 0x7fffff) >> 20, rest = a & 0xfffff; int e = (int)(a >> 23) - 120;
      if (rest > 0x80000 || (rest == 0x80000 && (keep & 1))) { if (++keep == 8) { keep = 0; ++e; } }
      if (e > 15 || (e == 15 && keep == 7)) return sign | 0x7e;
      return sign | (uint8_t)(e << 3) | (uint8_t)keep;
    }
    int main(int argc, char** argv) {
      long n = atol(argv[1]), badq = 0, badc = 0, nq = 0, nc = 0;
      for (long i = 0; i < n; ++i) {
        uint64_t r = xr(), r2 = xr();
        float b;
        switch (r & 3) {
          case 0: b = 0x1p-64f * (1.0f + (float)((r >> 8) & 0xffff) / 65536.0f); break;
          case 1: b = u2f(f2u(0x1p100f) - (uint32_t)((r >> 8) & 0xffff)); break;
          default: b = ldexpf(1.0f + (float)((r >> 8) & 0x7fffff) / 8388608.0f, (int)((r >> 40) % 165) - 64);
        }
        if (!(b >= 0x1p-64f && b <= 0x1p100f)) continue;
        float a;
        switch (r2 & 7) {
          case 0: a = u2f((uint32_t)((r2 >> 8) & 0x7fffff)); break;                     /* subnormal */
          case 1: a = u2f((uint32_t)((r2 >> 8) & 0x7fffffff)); break;                   /* any pattern */
          case 2: a = ldexpf(1.0f + (float)((r2 >> 8) & 0x7fffff) / 8388608.0f, (int)((r2 >> 40) % 30) - 126); break;
          case 3: {  /* beside an e4m3 rounding midpoint of the quotient */
            float m = ldexpf(1.0f + ((float)((r2 >> 16) % 16) + 0.5f) / 16.0f, (int)((r2 >> 8) % 19) - 10);
            a = u2f(f2u(m * b) + (int32_t)((r2 >> 24) % 9) - 4); break;
          }
          case 4: a = 0.0f; break;
          default: a = b * 448.0f * ((float)((r2 >> 8) & 0xffffff) / 16777216.0f);
        }
        if (!(fabsf(a) <= 448.0f * b * 1.0001f)) continue;
        if (r2 >> 63) a = -a;
        float rb = 1.0f / b, q = a * rb;
        float got = copysignf(fmaf(fmaf(-q, b, a), rb, q), a), want = a / b;
        ++nc; if (e4m3(got) != e4m3(want)) ++badc;
        if (fabsf(a) >= 0x1p-100f || a == 0.0f) { ++nq; if (f2u(got) != f2u(want)) ++badq; }
      }
      printf("%ld %ld %ld %ld\n", nc, badc, nq, badq);
      return 0;
    }
""")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_div_rn_matches_ieee_division(tmp_path):
    src = tmp_path / "div_rn.c"
    exe = tmp_path / "div_rn"
    src.write_text(_SRC)
    # -ffp-contract=off: a * rb must stay a rounded product, as in the device code
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(src), "-lm"], check=True)
    out = subprocess.run([str(exe), "30000000"], check=True, capture_output=True, text=True).stdout.split()
    nc, badc, nq, badq = map(int, out)
    assert nc > 20_000_000 and nq > 15_000_000
    assert badc == 0, f"{badc} e4m3 codes differ"
    assert badq == 0, f"{badq} quotients differ"
