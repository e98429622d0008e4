/*
 * Deterministic elementary functions shared bit-for-bit by host and device.
 *
 * The reference leaves exp, rsqrt, sin, cos and pow to each backend's native
 * FP32 library ("Matching a particular GPU's approximation of exp, rsqrt, sin
 * or cos is not a portability requirement",
 * docs/architecture/numerical-portability.md:3-6).  This build instead fixes
 * one implementation, written from textbook methods, so that the gfx950
 * kernels and the CPU contract restatement produce identical bits:
 *
 *  - exp: Cody-Waite reduction x = k*ln2 + r with ln2 split into a 29-bit
 *    head (k*head exact for |k| < 2^24) and a tail, then the Taylor series
 *    of exp(r) - 1 - r to degree 13 on |r| <= ln2/2 (truncation < 4e-18),
 *    and scaling by 2^k through the exponent field.
 *  - log: x = 2^e * m with m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(f),
 *    f = (m-1)/(m+1), atanh series to f^21 (|f| <= 0.1716).
 *  - pow (positive base only): exp(e * log(base)), used for the RoPE
 *    inverse frequencies before their rounding to binary32.
 *  - sin/cos: Cody-Waite reduction by pi/2 with a three-part split (each
 *    part 30 bits, so k*part is exact for |k| < 2^23), then the Taylor series
 *    of sin and cos on |r| <= pi/4 to degree 17/18.
 *
 * Every operation is a basic IEEE-754 operation (+, -, *, /, sqrt) or an
 * explicit fused multiply-add, so results do not depend on the compiler as
 * long as contraction is disabled (-ffp-contract=off on every compile line).
 * Binary32 entry points evaluate in binary64 and round once.
 */
#ifndef DL_MATH_H
#define DL_MATH_H

#include "dl_common.h"

#if defined(__HIPCC__)
#define DL_FMA(a, b, c) __builtin_fma((a), (b), (c))
#else
#include <math.h>
#define DL_FMA(a, b, c) fma((a), (b), (c))
#endif

#define DL_LN2_HI 0x1.62e42ffp-1
#define DL_LN2_LO -0x1.718432a1b0e26p-35
#define DL_LOG2E 0x1.71547652b82fep+0
#define DL_2_OVER_PI 0x1.45f306dc9c883p-1
#define DL_PIO2_1 0x1.921fb548p+0
#define DL_PIO2_2 -0x1.de973dc8p-31
#define DL_PIO2_3 -0x1.9d9cceba3f91fp-62
#define DL_TWO_PI 0x1.921fb54442d18p+2
/* 1.5 * 2^52: adding and subtracting it rounds a |v| < 2^51 to an integer
 * with ties to even. */
#define DL_ROUND_SHIFTER 0x1.8p52

DL_HD double dl_rint(double v) { return (v + DL_ROUND_SHIFTER) - DL_ROUND_SHIFTER; }

/* 2^k for -1022 <= k <= 1023 built from the exponent field. */
DL_HD double dl_pow2i(int k) { return dl_bits_to_f64((uint64_t)(k + 1023) << 52); }

DL_HD double dl_exp(double x) {
  if (x != x) return x;
  if (x > 709.782712893384) return dl_bits_to_f64(0x7ff0000000000000ull);
  if (x < -745.1332191019412) return 0.0;
  const double kd = dl_rint(x * DL_LOG2E);
  double r = DL_FMA(-kd, DL_LN2_HI, x); /* exact: Sterbenz */
  r = DL_FMA(-kd, DL_LN2_LO, r);
  /* q = (exp(r) - 1 - r) / r^2 = sum_{n>=2} r^(n-2) / n! */
  double q = 0x1.6124613a86d09p-33;            /* 1/13! */
  q = DL_FMA(q, r, 0x1.1eed8eff8d898p-29);     /* 1/12! */
  q = DL_FMA(q, r, 0x1.ae64567f544e4p-26);     /* 1/11! */
  q = DL_FMA(q, r, 0x1.27e4fb7789f5cp-22);     /* 1/10! */
  q = DL_FMA(q, r, 0x1.71de3a556c734p-19);     /* 1/9!  */
  q = DL_FMA(q, r, 0x1.a01a01a01a01ap-16);     /* 1/8!  */
  q = DL_FMA(q, r, 0x1.a01a01a01a01ap-13);     /* 1/7!  */
  q = DL_FMA(q, r, 0x1.6c16c16c16c17p-10);     /* 1/6!  */
  q = DL_FMA(q, r, 0x1.1111111111111p-7);      /* 1/5!  */
  q = DL_FMA(q, r, 0x1.5555555555555p-5);      /* 1/4!  */
  q = DL_FMA(q, r, 0x1.5555555555555p-3);      /* 1/3!  */
  q = DL_FMA(q, r, 0.5);
  const double u = DL_FMA(r * r, q, r);
  const double p = 1.0 + u;
  const int k = (int)kd;
  if (k > 1023) return (p * dl_pow2i(k - 1)) * 2.0;
  if (k < -1022) return (p * dl_pow2i(k + 1022)) * 0x1p-1022;
  return p * dl_pow2i(k);
}

DL_HD float dl_expf(float x) { return (float)dl_exp((double)x); }

/* Natural logarithm for finite x > 0. */
DL_HD double dl_log(double x) {
  int e = 0;
  uint64_t b = dl_f64_to_bits(x);
  if ((b >> 52) == 0) { /* subnormal */
    x = x * 0x1p54;
    e = -54;
    b = dl_f64_to_bits(x);
  }
  e += (int)((b >> 52) & 0x7ff) - 1023;
  double m = dl_bits_to_f64((b & 0x000fffffffffffffull) | 0x3ff0000000000000ull);
  if (m > 0x1.6a09e667f3bcdp+0) { /* sqrt(2) */
    m = m * 0.5;
    e += 1;
  }
  const double f = (m - 1.0) / (m + 1.0);
  const double s = f * f;
  double t = 1.0 / 21.0;
  t = DL_FMA(t, s, 1.0 / 19.0);
  t = DL_FMA(t, s, 1.0 / 17.0);
  t = DL_FMA(t, s, 1.0 / 15.0);
  t = DL_FMA(t, s, 1.0 / 13.0);
  t = DL_FMA(t, s, 1.0 / 11.0);
  t = DL_FMA(t, s, 1.0 / 9.0);
  t = DL_FMA(t, s, 1.0 / 7.0);
  t = DL_FMA(t, s, 1.0 / 5.0);
  t = DL_FMA(t, s, 1.0 / 3.0);
  const double f2 = f + f;
  const double logm = DL_FMA(f2 * s, t, f2);
  const double ed = (double)e;
  return DL_FMA(ed, DL_LN2_HI, DL_FMA(ed, DL_LN2_LO, logm));
}

/* base^e for finite base > 0, as exp(e * log(base)). */
DL_HD double dl_pow_pos(double base, double e) {
  if (e == 0.0) return 1.0;
  return dl_exp(e * dl_log(base));
}

/* sin and cos of x for |x| < 2^20. */
DL_HD void dl_sincos(double x, double* sin_out, double* cos_out) {
  const double kd = dl_rint(x * DL_2_OVER_PI);
  double r = DL_FMA(-kd, DL_PIO2_1, x);
  r = DL_FMA(-kd, DL_PIO2_2, r);
  r = DL_FMA(-kd, DL_PIO2_3, r);
  const double s = r * r;
  double ps = 0x1.952c77030ad4ap-49;        /* 1/17! */
  ps = DL_FMA(ps, s, -0x1.ae7f3e733b81fp-41); /* -1/15! */
  ps = DL_FMA(ps, s, 0x1.6124613a86d09p-33);  /* 1/13! */
  ps = DL_FMA(ps, s, -0x1.ae64567f544e4p-26); /* -1/11! */
  ps = DL_FMA(ps, s, 0x1.71de3a556c734p-19);  /* 1/9! */
  ps = DL_FMA(ps, s, -0x1.a01a01a01a01ap-13); /* -1/7! */
  ps = DL_FMA(ps, s, 0x1.1111111111111p-7);   /* 1/5! */
  ps = DL_FMA(ps, s, -0x1.5555555555555p-3);  /* -1/3! */
  const double sin_r = DL_FMA(r * s, ps, r);
  /* cos r = 1 - s * (1/2! - s/4! + s^2/6! - ... + s^8/18!) */
  double pc = 0x1.6827863b97d97p-53;          /* 1/18! */
  pc = DL_FMA(pc, s, -0x1.ae7f3e733b81fp-45); /* -1/16! */
  pc = DL_FMA(pc, s, 0x1.93974a8c07c9dp-37);  /* 1/14! */
  pc = DL_FMA(pc, s, -0x1.1eed8eff8d898p-29); /* -1/12! */
  pc = DL_FMA(pc, s, 0x1.27e4fb7789f5cp-22);  /* 1/10! */
  pc = DL_FMA(pc, s, -0x1.a01a01a01a01ap-16); /* -1/8! */
  pc = DL_FMA(pc, s, 0x1.6c16c16c16c17p-10);  /* 1/6! */
  pc = DL_FMA(pc, s, -0x1.5555555555555p-5);  /* -1/4! */
  pc = DL_FMA(pc, s, 0.5);                    /* 1/2! */
  const double cos_r = DL_FMA(-s, pc, 1.0);
  const int quadrant = (int)((int64_t)kd & 3);
  double sv, cv;
  switch (quadrant) {
    case 0: sv = sin_r; cv = cos_r; break;
    case 1: sv = cos_r; cv = -sin_r; break;
    case 2: sv = -sin_r; cv = -cos_r; break;
    default: sv = -cos_r; cv = sin_r; break;
  }
  *sin_out = sv;
  *cos_out = cv;
}

#endif /* DL_MATH_H */
