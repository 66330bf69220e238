// Deterministic fp32 exp/log used by the router so that its scores are reproducible
// bit-for-bit by a plain C restatement on the CPU. Every step is an IEEE-754 operation with a
// single correctly-rounded result (mul, add, fma, div, rint, ldexp), written out explicitly;
// the translation unit that includes this file is compiled with floating-point contraction off.
//
// exp: Cody-Waite reduction x = n*ln2 + r, |r| <= ln2/2, then the degree-7 Taylor polynomial of
//      e^r in Horner form, then scaling by 2^n. Results below 2^-125 are flushed to +0 so that
//      no subnormal rounding enters.
// log: x = m*2^e with m in [sqrt(1/2), sqrt(2)), log(m) = 2*atanh(s), s=(m-1)/(m+1), odd series
//      to s^13.
#pragma once
#include "common.h"

#define MI355_LN2_HI 0.693145751953125f
#define MI355_LN2_LO 1.428606765330187e-06f

MI355_DEV float det_expf(float x) {
  if (x != x) return x;
  if (x > 88.75f) return __builtin_inff();
  if (x < -87.0f) return 0.0f;
  float n = rintf(x * 1.44269504088896341f);
  float r = fmaf(-n, MI355_LN2_HI, x);
  r = fmaf(-n, MI355_LN2_LO, r);
  float p = 1.98412698e-04f;             // 1/5040
  p = fmaf(p, r, 1.38888889e-03f);       // 1/720
  p = fmaf(p, r, 8.33333377e-03f);       // 1/120
  p = fmaf(p, r, 4.16666679e-02f);       // 1/24
  p = fmaf(p, r, 1.66666672e-01f);       // 1/6
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

// Natural log for finite x > 0 (normal range); returns -inf for 0, NaN for negatives.
MI355_DEV float det_logf(float x) {
  if (!(x > 0.0f)) return x == 0.0f ? -__builtin_inff() : __builtin_nanf("");
  if (x == __builtin_inff()) return x;
  uint32_t bits = __float_as_uint(x);
  int e = (int)((bits >> 23) & 0xff) - 127;
  float m = __uint_as_float((bits & 0x7fffffu) | 0x3f800000u);
  if (m > 1.41421356f) { m = m * 0.5f; e += 1; }
  float f = m - 1.0f;
  float s = f / (2.0f + f);
  float z = s * s;
  float p = 0.15384615384615385f;        // 2/13
  p = fmaf(p, z, 0.18181818181818182f);  // 2/11
  p = fmaf(p, z, 0.22222222222222221f);  // 2/9
  p = fmaf(p, z, 0.2857142857142857f);   // 2/7
  p = fmaf(p, z, 0.4f);                  // 2/5
  p = fmaf(p, z, 0.6666666666666666f);   // 2/3
  p = fmaf(p, z, 2.0f);
  float lm = s * p;
  float ef = (float)e;
  return fmaf(ef, MI355_LN2_HI, fmaf(ef, MI355_LN2_LO, lm));
}
