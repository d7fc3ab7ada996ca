// expf with the results of glibc's expf (the libm call libbnneon's scalar SiLU makes: silu_s, src/v24_f32.c:160, in
// the squeeze-excitation's first FC). glibc >= 2.27 computes expf by the published table method of ARM's optimized
// routines (Szabolcs Nagy): x N / ln 2 = k + r, |r| <= 1/2, N = 32; 2^(k/N) from a 32-entry table of 2^(i/N) whose
// entries carry the exponent adjustment -(i << 47); 2^(r/N) by a cubic; the product rounded once to float. Its
// results are correctly rounded except within ~0.002 ulp of a midpoint, so a correctly rounded expf would differ from
// it in about 0.3% of arguments: the steps are restated here, with the multiply-adds fused where GCC fuses them when
// it builds glibc for an FMA target (AArch64, and the x86-64 FMA variant that an FMA host dispatches to).
//
// Usable from device and host code (the host build checks it against the C library's expf for every float).
#ifndef BNH_EXPF_H
#define BNH_EXPF_H
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define BNH_HD __host__ __device__ __forceinline__
#else
#define BNH_HD static inline
#endif

// 2^(i/32) rounded to double, as bits, minus i << 47 (so that adding k << 47 for k = i + 32 m gives 2^(k/32))
#define BNH_EXP2F_TAB                                                                                           \
  {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,                \
   0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,                \
   0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,                \
   0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,                \
   0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,                \
   0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,                \
   0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,                \
   0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

BNH_HD float bnh_expf(float x) {
  const uint64_t tab[32] = BNH_EXP2F_TAB;
  const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
               c2 = 0x1.62e42ff0c52d6p-1 / 32;
  uint32_t ux;
  memcpy(&ux, &x, 4);
  const uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= (0x42b00000u >> 20)) {  // |x| >= 88 or NaN
    if (ux == 0xff800000u) return 0.f;
    if (abstop >= (0x7f800000u >> 20)) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.f;
  }
  const double xd = (double)x;
  const double kt = __builtin_fma(inv_ln2_n, xd, shift);  // round(x N / ln 2) in the low bits (ties to even)
  uint64_t ki;
  memcpy(&ki, &kt, 8);
  const double kd = kt - shift;
  const double r = __builtin_fma(inv_ln2_n, xd, -kd);
  uint64_t t = tab[ki % 32] + (ki << 47);
  double s;
  memcpy(&s, &t, 8);
  const double z = __builtin_fma(c0, r, c1);
  const double r2 = r * r;
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

#endif
