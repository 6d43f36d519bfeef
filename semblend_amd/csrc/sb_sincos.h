// sin and cos in double precision for RoPE angles, written for a small register footprint.
//
// RoPE rotates by angles x = delta * inv_freq (fp32), and the kernels round sin(x) and cos(x)
// to fp32. Evaluated in double precision and rounded once, the fp32 values are the correctly
// rounded ones except when the exact value lies within about 1e-16 (relative) of a rounding
// midpoint. A general-purpose double sincos also handles arguments up to 1e308, which takes
// a wide reduction and many live registers; this one is limited to |x| < 2^32 (RoPE angles are
// an int32 position, or a difference of two, times an inverse frequency <= 1; the difference
// of an int32 target and a valid, non-negative donor position stays below 2^32) and keeps
// about a dozen doubles live.
//
// Method: Cody-Waite argument reduction (W. J. Cody and W. Waite, "Software Manual for the
// Elementary Functions", 1980): k = rint(x * 2/pi), r = x - k * pi/2 with pi/2 split into three
// parts of 21 significant bits and a double tail, each subtracted with one fused multiply-add
// (k * part is exact for |k| < 2^32, which |x| < 2^32 keeps: |k| <= |x| 2/pi + 1/2). Then the Taylor series of sin and cos on
// |r| <= pi/4 (+ rounding slack), through r^17 and r^18, whose first omitted terms are below
// 5e-18 and 4e-21 there, and the quadrant k mod 4 picks and negates the pair.
//
// Compiled for the host as well, so that a CPU test can compare it with the C library over
// every angle the kernels form.
#pragma once

#if defined(__HIPCC__)
#define SB_HD __host__ __device__
#else
#define SB_HD
#endif

namespace sb {

SB_HD inline void sincos_cw(double x, double* s, double* c) {
  // pi/2 = P1 + P2 + P3 + P4 (P1..P3: 21 significant bits each; |P4| < 2^-65)
  constexpr double kP1 = 0x1.921fb00000000p+0;
  constexpr double kP2 = 0x1.5110b00000000p-22;
  constexpr double kP3 = 0x1.1846a00000000p-44;
  constexpr double kP4 = -0x1.d9cceba3f91f2p-66;
  constexpr double kTwoOverPi = 0x1.45f306dc9c883p-1;
  const double k = __builtin_rint(x * kTwoOverPi);
  double r = __builtin_fma(-k, kP1, x);
  r = __builtin_fma(-k, kP2, r);
  r = __builtin_fma(-k, kP3, r);
  r = __builtin_fma(-k, kP4, r);
  const double r2 = r * r;
  // sin r = r + r^3 (-1/3! + r^2 (1/5! - ...)), cos r = 1 + r^2 (-1/2! + r^2 (1/4! - ...))
  double sp = 0x1.952c77030ad4ap-49;           //  1/17!
  sp = __builtin_fma(sp, r2, -0x1.ae7f3e733b81fp-41);  // -1/15!
  sp = __builtin_fma(sp, r2, 0x1.6124613a86d09p-33);   //  1/13!
  sp = __builtin_fma(sp, r2, -0x1.ae64567f544e4p-26);  // -1/11!
  sp = __builtin_fma(sp, r2, 0x1.71de3a556c734p-19);   //  1/9!
  sp = __builtin_fma(sp, r2, -0x1.a01a01a01a01ap-13);  // -1/7!
  sp = __builtin_fma(sp, r2, 0x1.1111111111111p-7);    //  1/5!
  sp = __builtin_fma(sp, r2, -0x1.5555555555555p-3);   // -1/3!
  const double sn = __builtin_fma(sp * r2, r, r);
  double cp = -0x1.6827863b97d97p-53;          // -1/18!
  cp = __builtin_fma(cp, r2, 0x1.ae7f3e733b81fp-45);   //  1/16!
  cp = __builtin_fma(cp, r2, -0x1.93974a8c07c9dp-37);  // -1/14!
  cp = __builtin_fma(cp, r2, 0x1.1eed8eff8d898p-29);   //  1/12!
  cp = __builtin_fma(cp, r2, -0x1.27e4fb7789f5cp-22);  // -1/10!
  cp = __builtin_fma(cp, r2, 0x1.a01a01a01a01ap-16);   //  1/8!
  cp = __builtin_fma(cp, r2, -0x1.6c16c16c16c17p-10);  // -1/6!
  cp = __builtin_fma(cp, r2, 0x1.5555555555555p-5);    //  1/4!
  cp = __builtin_fma(cp, r2, -0.5);                     // -1/2!
  const double cs = __builtin_fma(cp, r2, 1.0);
  // x = k pi/2 + r: quadrant q = k mod 4 (two's complement keeps it right for k < 0)
  const int q = static_cast<int>(static_cast<long long>(k) & 3);
  const double a = (q & 1) ? cs : sn;  // |sin x|
  const double b = (q & 1) ? sn : cs;  // |cos x|
  *s = (q & 2) ? -a : a;
  *c = ((q + 1) & 2) ? -b : b;
}

}  // namespace sb
