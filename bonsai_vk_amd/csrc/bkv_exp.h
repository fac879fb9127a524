// bkv_exp.h - exp(x) of a float, correctly rounded to float, by a 32-entry table (the decode and
// prefill kernels' e = exp(s*scale - max)).
#pragma once

#include <hip/hip_runtime.h>

namespace bkv {

// 2^(j/32), j = 0..31, correctly rounded to fp64
static __constant__ double kExp2Tab[32] = {
    0x1.0000000000000p+0, 0x1.059b0d3158574p+0, 0x1.0b5586cf9890fp+0, 0x1.11301d0125b51p+0,
    0x1.172b83c7d517bp+0, 0x1.1d4873168b9aap+0, 0x1.2387a6e756238p+0, 0x1.29e9df51fdee1p+0,
    0x1.306fe0a31b715p+0, 0x1.371a7373aa9cbp+0, 0x1.3dea64c123422p+0, 0x1.44e086061892dp+0,
    0x1.4bfdad5362a27p+0, 0x1.5342b569d4f82p+0, 0x1.5ab07dd485429p+0, 0x1.6247eb03a5585p+0,
    0x1.6a09e667f3bcdp+0, 0x1.71f75e8ec5f74p+0, 0x1.7a11473eb0187p+0, 0x1.82589994cce13p+0,
    0x1.8ace5422aa0dbp+0, 0x1.93737b0cdc5e5p+0, 0x1.9c49182a3f090p+0, 0x1.a5503b23e255dp+0,
    0x1.ae89f995ad3adp+0, 0x1.b7f76f2fb5e47p+0, 0x1.c199bdd85529cp+0, 0x1.cb720dcef9069p+0,
    0x1.d5818dcfba487p+0, 0x1.dfc97337b9b5fp+0, 0x1.ea4afa2a490dap+0, 0x1.f50765b6e4540p+0,
};

// v = fma(p, r, c) with c an SGPR pair (the compiler's accumulator form would move each constant
// into VGPRs first)
__device__ __forceinline__ double fma_sc(double p, double r, double c) {
  double v;
  asm("v_fma_f64 %0, %1, %2, %3" : "=v"(v) : "v"(p), "v"(r), "s"(c));
  return v;
}

// exp of a float argument, correctly rounded to float: the value of (float)exp((double)x), as
// exp_cr, by a table. x = (k/32) ln2 + r with |r| <= ln2/64 (ln2/32 split so that k*hi is exact for
// |k| < 2^12), exp(r) by its degree-5 Taylor polynomial in fp64 (truncation < 2^-48.6), times
// t2[k mod 32] = 2^((k mod 32)/32) and 2^floor(k/32), rounded once to float. When the fp64 value lies
// within 64 units of its last place of a float rounding boundary (the error is below 16), or x is
// outside (-87, 88), the library fp64 exp decides. t2: kExp2Tab in LDS. Checked on the host against
// (float)exp((double)x) over every float in [-104, 89] (tests/test_exp_table.py runs a stride of it).
__device__ __forceinline__ float exp_cr_t(float xf, const double *t2) {
  const float kf = __builtin_rintf(xf * 46.16624130844683f);      // 32 / ln2
  const int k = (int)kf;
  const double x = xf, kd = kf;
  double r = fma(-kd, 0x1.62e42fefa3800p-6, x);                     // ln2/32, 41 bits
  r = fma(-kd, 0x1.ef35793c76730p-50, r);                           // the rest of ln2/32
  double p = fma_sc(r, 0x1.1111111111111p-7, 0x1.5555555555555p-5); // 1/120 r + 1/24
  p = fma_sc(p, r, 0x1.5555555555555p-3);
  p = fma_sc(p, r, 0.5);
  p = fma_sc(p, r, 1.0);
  p = fma_sc(p, r, 1.0);
  const double y = ldexp(p * t2[k & 31], k >> 5);
  const long long low = (long long)(__double_as_longlong(y) & 0x1FFFFFFFll) - 0x10000000ll;
  float res = (float)y;
  if (!(xf > -87.0f && xf < 88.0f) || (low >= -64 && low <= 64)) res = (float)exp(x);
  return res;
}

// The same value in two steps, for callers that form many exps at once: exp_t_fast is the table
// path alone, branch-free (so independent calls interleave and their table reads overlap), and
// sets `slow` where exp_cr_t would let the library decide; exp_t_slow is that decision (x <= -104
// rounds to +0 without the library: exp(-104) < 2^-150).
__device__ __forceinline__ float exp_t_fast(float xf, const double *t2, bool &slow) {
  const float kf = __builtin_rintf(xf * 46.16624130844683f);
  const int k = (int)kf;
  const double x = xf, kd = kf;
  double r = fma(-kd, 0x1.62e42fefa3800p-6, x);
  r = fma(-kd, 0x1.ef35793c76730p-50, r);
  double p = fma_sc(r, 0x1.1111111111111p-7, 0x1.5555555555555p-5);
  p = fma_sc(p, r, 0x1.5555555555555p-3);
  p = fma_sc(p, r, 0.5);
  p = fma_sc(p, r, 1.0);
  p = fma_sc(p, r, 1.0);
  const double y = ldexp(p * t2[k & 31], k >> 5);
  const long long low = (long long)(__double_as_longlong(y) & 0x1FFFFFFFll) - 0x10000000ll;
  slow = !(xf > -87.0f && xf < 88.0f) || (low >= -64 && low <= 64);
  return (float)y;
}
__device__ __forceinline__ float exp_t_slow(float xf) {
  return xf <= -104.0f ? 0.0f : (float)exp((double)xf);
}

}  // namespace bkv
