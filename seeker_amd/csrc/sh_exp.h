// f64 exp for non-positive arguments, used by the acceptance kernels' softmax
// statistics and inverse-CDF draws (every vocab entry of every row goes through
// it, so its cost sets those kernels' speed).
//
// Method: Tang's table-driven reduction (P. T. P. Tang, "Table-driven
// implementation of the exponential function in IEEE floating-point
// arithmetic", ACM TOMS 15(2), 1989) with a 64-entry table:
//   y = n ln2/64 + r, n = rint(64 y / ln2), |r| <= ln2/128 (+ rounding),
//   exp(y) = 2^(n >> 6) * 2^((n & 63)/64) * e^r,
// r computed exactly by a Cody-Waite split of ln2/64 with fused multiply-adds
// (|n| < 2^17, so y - n * kLn2o64Hi needs no more than 53 bits), e^r - 1 by its
// degree-6 Taylor polynomial (truncation < 2^-60 relative), 2^(j/64) correctly
// rounded to f64. Result error about 1 ulp at most; arguments below -746 (and
// -inf) return 0; denormal results are rounded once, by ldexp.
#pragma once

#include <hip/hip_runtime.h>

// 2^(j/64), j = 0..63, each correctly rounded to f64.
#define SH_EXP2_TABLE_64 \
  { \
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0, \
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0, \
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0, \
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0, \
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0, \
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0, \
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0, \
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0, \
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0, \
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0, \
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0, \
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0, \
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0, \
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0, \
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0, \
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0, \
  }

constexpr double kExp64OverLn2 = 0x1.71547652b82fep+6;
constexpr double kLn2o64Hi = 0x1.62e42fefa39efp-7;
constexpr double kLn2o64Lo = 0x1.abc9e3b39803fp-62;

// 1.5 * 2^52: adding it rounds to an integer held in the low mantissa bits.
constexpr double kRoundShift = 0x1.8p52;

// exp(y), y <= 0; tab holds the SH_EXP2_TABLE_64 values (in LDS on the device).
// n = rint(64 y / ln2) comes from one fused multiply-add with kRoundShift (its
// low 32 bits are n in two's complement, |n| < 2^17), with no conversions.
__host__ __device__ inline double sh_exp_neg(double y, const double* tab) {
  y = fmax(y, -746.0);
  const double kd = fma(y, kExp64OverLn2, kRoundShift);
  const double t = kd - kRoundShift;
  const int n = (int)(uint32_t)__builtin_bit_cast(unsigned long long, kd);
  const double r = fma(-t, kLn2o64Lo, fma(-t, kLn2o64Hi, y));
  double q = fma(r, 1.0 / 720.0, 1.0 / 120.0);
  q = fma(q, r, 1.0 / 24.0);
  q = fma(q, r, 1.0 / 6.0);
  q = fma(q, r, 0.5);
  q = fma(q, r, 1.0);
  const double tj = tab[n & 63];
  return ldexp(fma(tj, q * r, tj), n >> 6);
}
