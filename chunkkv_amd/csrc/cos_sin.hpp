// cos and sin of an fp32 angle, each rounded once to fp32 from an fp64 evaluation: the values
// (float)cos((double)x) and (float)sin((double)x) that the rotary reference tables hold.
//
// Method (textbook Cody-Waite reduction + Taylor series, all in IEEE fp64):
//   k = rint(x * 2/pi);  r = (x - k * P1) - k * P2   with P1 + P2 = pi/2 to 107 bits, each step
//   one fused multiply-add (x - k * P1 is exact: the product is exact inside the fma and the
//   difference has fewer than 53 significant bits for |k| < 2^31);
//   sin r = r + r z (-1/3! + z (1/5! - ... + z / 17!)),  cos r = 1 - z (1/2! - z (1/4! - ... - z / 18!)),
//   z = r^2, |r| <= pi/4 (truncation error below 2^-62); the quadrant k mod 4 picks and negates.
// For |x| < 2^31 (every angle an int32 position times an inverse frequency <= 1 can give) the
// fp32 results equal glibc's (float)cos/sin((double)x) bit for bit for every float, +-0 and
// subnormals included: checked exhaustively by tests/test_cos_sin.py. Larger or non-finite
// angles return false and the caller uses the library sincos.
//
// The header compiles for the device (hipcc) and the host (g++), so that the exhaustive check
// runs this same source on the CPU.
#pragma once

#include <cmath>

#if defined(__HIPCC__)
#define CKV_HOST_DEVICE __host__ __device__
#else
#define CKV_HOST_DEVICE
#endif

namespace ckv {

// Branch-free: for |x| >= 2^31, infinities and NaN it returns false and c, s are unspecified.
CKV_HOST_DEVICE inline bool cos_sin_fast(float x, float& c, float& s) {
  const bool ok = std::fabs(x) < 0x1p31f;  // false for NaN too
  const double xd = ok ? (double)x : 0.0;
  const double k = std::rint(xd * 0x1.45f306dc9c883p-1);  // 2/pi
  double r = std::fma(-k, 0x1.921fb54442d18p+0, xd);      // pi/2, high part
  r = std::fma(-k, 0x1.1a62633145c07p-54, r);             // pi/2, next 53 bits
  r = k == 0.0 ? xd : r;                                  // keeps the sign of -0
  const double z = r * r;
  double sp = 1.0 / 355687428096000.0;  // 1/17!
  sp = std::fma(sp, z, -1.0 / 1307674368000.0);
  sp = std::fma(sp, z, 1.0 / 6227020800.0);
  sp = std::fma(sp, z, -1.0 / 39916800.0);
  sp = std::fma(sp, z, 1.0 / 362880.0);
  sp = std::fma(sp, z, -1.0 / 5040.0);
  sp = std::fma(sp, z, 1.0 / 120.0);
  sp = std::fma(sp, z, -1.0 / 6.0);
  double sn = std::fma(r * z, sp, r);
  sn = xd == 0.0 ? xd : sn;  // sin(+-0) = +-0
  double cp = 1.0 / 6402373705728000.0;  // 1/18!
  cp = std::fma(cp, z, -1.0 / 20922789888000.0);
  cp = std::fma(cp, z, 1.0 / 87178291200.0);
  cp = std::fma(cp, z, -1.0 / 479001600.0);
  cp = std::fma(cp, z, 1.0 / 3628800.0);
  cp = std::fma(cp, z, -1.0 / 40320.0);
  cp = std::fma(cp, z, 1.0 / 720.0);
  cp = std::fma(cp, z, -1.0 / 24.0);
  cp = std::fma(cp, z, 0.5);
  const double cs = std::fma(-z, cp, 1.0);
  const int q = (int)k & 3;  // k mod 4, also for negative k (two's complement)
  double cc = (q & 1) ? -sn : cs;
  double ss = (q & 1) ? cs : sn;
  cc = (q & 2) ? -cc : cc;
  ss = (q & 2) ? -ss : ss;
  c = (float)cc;
  s = (float)ss;
  return ok;
}

}  // namespace ckv
