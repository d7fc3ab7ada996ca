// powf with the results of glibc's powf (the libm call of GEM_A's final power, src/rt_ops_dot.c:452). glibc >= 2.28
// computes powf by the published method of ARM's optimized routines (Szabolcs Nagy): log2(x) in double from a
// 16-entry table of (1/c, log2 c) for subintervals of [0x1.66p-1, 0x1.66p0) and a degree-5 polynomial in
// r = z/c - 1; y log2(x) in double; 2^(y log2 x) by the 32-entry exp2 table (the one expf uses) and a cubic; the
// product rounded once to float (about 0.82 ulp at worst, so a correctly rounded powf would differ from it now and
// then). The steps are restated here with the multiply-adds fused where GCC fuses them when it builds glibc for an
// FMA target (AArch64; the x86-64 FMA variant an FMA host dispatches to), and the special cases of its entry.
//
// Usable from device and host code (tests/native/powf_check.c checks it against the C library's powf).
#ifndef BNH_POWF_H
#define BNH_POWF_H
#include <stdint.h>
#include <string.h>

#include "bnh_expf.h"

// 1/c and log2(c) per subinterval (c near its centre; 1/c chosen so that z/c - 1 is exact)
#define BNH_POWF_LOG2_TAB                                                                                       \
  {{0x1.661ec79f8f3bep+0, -0x1.efec65b963019p-2}, {0x1.571ed4aaf883dp+0, -0x1.b0b6832d4fca4p-2},              \
   {0x1.49539f0f010bp+0, -0x1.7418b0a1fb77bp-2},  {0x1.3c995b0b80385p+0, -0x1.39de91a6dcf7bp-2},              \
   {0x1.30d190c8864a5p+0, -0x1.01d9bf3f2b631p-2}, {0x1.25e227b0b8eap+0, -0x1.97c1d1b3b7afp-3},                \
   {0x1.1bb4a4a1a343fp+0, -0x1.2f9e393af3c9fp-3}, {0x1.12358f08ae5bap+0, -0x1.960cbbf788d5cp-4},              \
   {0x1.0953f419900a7p+0, -0x1.a6f9db6475fcep-5}, {0x1p+0, 0x0p+0},                                          \
   {0x1.e608cfd9a47acp-1, 0x1.338ca9f24f53dp-4},  {0x1.ca4b31f026aap-1, 0x1.476a9543891bap-3},                \
   {0x1.b2036576afce6p-1, 0x1.e840b4ac4e4d2p-3},  {0x1.9c2d163a1aa2dp-1, 0x1.40645f0c6651cp-2},               \
   {0x1.886e6037841edp-1, 0x1.88e9c2c1b9ff8p-2},  {0x1.767dcf5534862p-1, 0x1.ce0a44eb17bccp-2}}

BNH_HD float bnh_f_from(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
BNH_HD uint32_t bnh_u_from(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

// 0: y is not an integer; 1: an odd integer; 2: an even integer (iy: a nonzero finite float's bits)
BNH_HD int bnh_powf_checkint(uint32_t iy) {
  const int e = iy >> 23 & 0xff;
  if (e < 0x7f) return 0;
  if (e > 0x7f + 23) return 2;
  if (iy & ((1u << (0x7f + 23 - e)) - 1)) return 0;
  if (iy & (1u << (0x7f + 23 - e))) return 1;
  return 2;
}
BNH_HD int bnh_powf_zeroinfnan(uint32_t ix) { return 2 * ix - 1 >= 2u * 0x7f800000 - 1; }

BNH_HD float bnh_powf(float x, float y) {
  const double tab[16][2] = BNH_POWF_LOG2_TAB;
  const double A0 = 0x1.27616c9496e0bp-2, A1 = -0x1.71969a075c67ap-2, A2 = 0x1.ec70a6ca7baddp-2,
               A3 = -0x1.7154748bef6c8p-1, A4 = 0x1.71547652ab82bp0;
  const uint64_t etab[32] = BNH_EXP2F_TAB;
  const double C0 = 0x1.c6af84b912394p-5, C1 = 0x1.ebfce50fac4f3p-3, C2 = 0x1.62e42ff0c52d6p-1;
  const double shift = 0x1.8p+52 / 32;
  uint32_t sign_bias = 0;
  uint32_t ix = bnh_u_from(x);
  const uint32_t iy = bnh_u_from(y);
  if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u || bnh_powf_zeroinfnan(iy)) {
    // x < 0x1p-126 or inf or NaN, or y 0, inf or NaN
    if (bnh_powf_zeroinfnan(iy)) {
      if (2 * iy == 0) return (ix & 0x7fc00000u) == 0x7f800000u && (ix & 0x3fffffu) ? x + y : 1.0f;
      if (ix == 0x3f800000u) return (iy & 0x7fc00000u) == 0x7f800000u && (iy & 0x3fffffu) ? x + y : 1.0f;
      if (2 * ix > 2u * 0x7f800000u || 2 * iy > 2u * 0x7f800000u) return x + y;
      if (2 * ix == 2 * 0x3f800000u) return 1.0f;
      if ((2 * ix < 2 * 0x3f800000u) == !(iy & 0x80000000u)) return 0.0f;  // |x| < 1, y = inf or |x| > 1, y = -inf
      return y * y;
    }
    if (bnh_powf_zeroinfnan(ix)) {
      float x2 = x * x;
      if ((ix & 0x80000000u) && bnh_powf_checkint(iy) == 1) x2 = -x2;
      return (iy & 0x80000000u) ? 1 / x2 : x2;
    }
    // x and y nonzero finite
    if (ix & 0x80000000u) {
      const int yint = bnh_powf_checkint(iy);
      if (yint == 0) return (x - x) / (x - x);  // invalid: NaN
      if (yint == 1) sign_bias = 1u << (5 + 11);
      ix &= 0x7fffffffu;
    }
    if (ix < 0x00800000u) {  // subnormal x: normalised, its exponent taken below the table's
      ix = bnh_u_from(bnh_f_from(ix) * 0x1p23f);
      ix &= 0x7fffffffu;
      ix -= 23u << 23;
    }
  }
  // log2(x) = log1p(z / c - 1) / ln 2 + log2(c) + k, x = 2^k z, z in [0x1.66p-1, 0x1.66p0)
  const uint32_t tmp = ix - 0x3f330000u;
  const int i = (int)((tmp >> (23 - 4)) % 16);
  const uint32_t top = tmp & 0xff800000u;
  const uint32_t iz = ix - top;
  const int k = (int32_t)top >> 23;
  const double invc = tab[i][0], logc = tab[i][1];
  const double z = (double)bnh_f_from(iz);
  const double r = __builtin_fma(z, invc, -1.0);
  const double y0 = logc + (double)k;
  const double r2 = r * r;
  double yl = __builtin_fma(A0, r, A1);
  const double p = __builtin_fma(A2, r, A3);
  const double r4 = r2 * r2;
  double q = __builtin_fma(A4, r, y0);
  q = __builtin_fma(p, r2, q);
  yl = __builtin_fma(yl, r4, q);
  const double ylogx = (double)y * yl;
  uint64_t ub;
  memcpy(&ub, &ylogx, 8);
  if ((ub >> 47 & 0xffff) >= (0x405f800000000000ull >> 47)) {  // |y log2 x| >= 126
    if (ylogx > 0x1.fffffffd1d571p+6) return sign_bias ? -0x1p97f * 0x1p97f : 0x1p97f * 0x1p97f;
    if (ylogx <= -150.0) return sign_bias ? -0x1p-95f * 0x1p-95f : 0x1p-95f * 0x1p-95f;
  }
  // 2^(y log2 x) = 2^(kk / 32) 2^rr, |rr| <= 1/64
  double kd = ylogx + shift;
  uint64_t ki;
  memcpy(&ki, &kd, 8);
  kd -= shift;
  const double rr = ylogx - kd;
  uint64_t t = etab[ki % 32];
  t += (ki + sign_bias) << (52 - 5);
  double s;
  memcpy(&s, &t, 8);
  const double zz = __builtin_fma(C0, rr, C1);
  const double rr2 = rr * rr;
  double ye = __builtin_fma(C2, rr, 1.0);
  ye = __builtin_fma(zz, rr2, ye);
  ye = ye * s;
  return (float)ye;
}

#endif
