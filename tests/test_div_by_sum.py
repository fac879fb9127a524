"""The exact prefill's quotient p = e / sum without a division (div_by_sum in
bonsai_vk_amd/csrc/bkv_prefill.hip) restated in C and checked against the correctly rounded fp32
quotient (float)((double)e / sum) (exact: a double-precision quotient rounded to fp32 is the
correctly rounded fp32 quotient), which is what the reference's p16 = f16(e / sum) rounds
(runtime_vk/attn_vk.h:190-200). The steps: q0 = e * rs with rs = fp32(1/sum), then twice
q = q + fma(-sum, q, e) * rs. Inputs: sum in [1, 2^18) with random significands (a softmax sum
reaches the key count: past 2^15 at 32K keys, 2^17 at the longest contexts the workspace takes) and 0 <= e <= sum
(a softmax sum includes its maximum's e = 1), spread over every binade of e and over e close to sum,
and sums whose significands are all ones or just above a power of two.
Below 2^-26 the quotient rounds to an fp16 zero whatever its last bits, so only the fp16 value is
compared there."""
import os
import subprocess
import tempfile

SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
static uint64_t st = 0x9E3779B97F4A7C15ull;
static uint64_t rnd(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float div_by_sum(float e, float s, float rs) {
  const float q0 = e * rs;
  const float q1 = fmaf(fmaf(-s, q0, e), rs, q0);
  return fmaf(fmaf(-s, q1, e), rs, q1);
}
int main(int argc, char **argv) {
  const long n = atol(argv[1]);
  long bad = 0;
  for (long i = 0; i < n; ++i) {
    const float s = u2f(0x3F800000u + (uint32_t)(rnd() % (18u << 23)));
    const uint64_t r = rnd();
    float e;
    switch (r & 3) {
      case 0: e = s * (float)((r >> 8) & 0xFFFFFF) * 0x1p-24f; break;          /* uniform in [0, s) */
      case 1: e = u2f(f2u(s) - (uint32_t)((r >> 8) & 0xFF)); break;   /* just below s */
      default: e = u2f((uint32_t)((r >> 8) % 0x3F800001u)); break;           /* every binade of [0, 1] */
    }
    if (e > s) e = s;
    const float q = div_by_sum(e, s, 1.0f / s);
    const float ref = (float)((double)e / (double)s);
    if (ref > 0x1p-26f ? q != ref : q > 0x1p-26f) {
      if (bad++ < 5) printf("e=%a s=%a q=%a ref=%a\n", e, s, q, ref);
    }
  }
  /* sums whose significands are all ones or just above a power of two (1/sum closest to a rounding
     boundary), against every 9973rd float of e in [2^-31, min(1, sum)] */
  for (int k = 0; k < 18; ++k)
    for (uint32_t m = 0; m < 16; ++m) {
      const float s = u2f(((127u + k) << 23) | (m < 8 ? 0x7FFFFFu - m : m - 8));
      for (uint32_t eb = 0x30000000u; eb <= 0x3F800000u && u2f(eb) <= s; eb += 9973) {
        const float e = u2f(eb);
        const float q = div_by_sum(e, s, 1.0f / s), ref = (float)((double)e / (double)s);
        if (q != ref && bad++ < 5) printf("e=%a s=%a q=%a ref=%a\n", e, s, q, ref);
      }
    }
  printf("%ld\n", bad);
  return 0;
}
"""


def test_div_by_sum_is_the_correctly_rounded_quotient():
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "t.c"), os.path.join(d, "t")
        with open(src, "w") as f:
            f.write("#include <stdlib.h>\n" + SRC)
        subprocess.run(["gcc", "-O2", "-o", exe, src, "-lm"], check=True)
        out = subprocess.run([exe, os.environ.get("BKV_DIV_CASES", "20000000")], check=True,
                             capture_output=True, text=True).stdout.split()
        assert out[-1] == "0", out
