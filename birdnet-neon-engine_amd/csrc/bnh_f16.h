// fp16 device helpers shared by the fp16 kernels: AArch64 fp16 semantics on gfx950's native fp16 instructions
// (v_fma_f16 / v_add_f16 / v_mul_f16 round once to nearest even and keep denormals, as FPCR.FZ16 = 0).
#ifndef BNH_F16_H
#define BNH_F16_H
#include "bnh_num.h"

typedef _Float16 h16;

BNH_DEV uint16_t hbits(h16 x) { return __builtin_bit_cast(uint16_t, x); }
BNH_DEV h16 hfrom(uint16_t u) { return __builtin_bit_cast(h16, u); }
BNH_DEV bool hnan(h16 x) { return x != x; }
BNH_DEV h16 hfma(h16 a, h16 b, h16 c) { return __builtin_fmaf16(a, b, c); }
// fp32 -> fp16, round to nearest even, of a value that has already been rounded to fp32 (FCVT h, s after an fp32
// operation). The empty asm pins the fp32 result in a register: without it the compiler may fold the producing
// fp32 FMA / add and this conversion into one v_fma_mix*_f16, a single rounding straight to fp16.
BNH_DEV h16 f2h(float y) {
  __asm__("" : "+v"(y));
  return (h16)y;
}
// FMAX / FMIN on fp16 (NaN-propagating, +0 above -0)
BNH_DEV h16 hmax(h16 a, h16 b) {
  if (hnan(a) || hnan(b)) return hfrom(0x7e00);
  if (a == (h16)0 && b == (h16)0) return hfrom((uint16_t)(hbits(a) & hbits(b)));
  return a > b ? a : b;
}
BNH_DEV h16 hmin(h16 a, h16 b) {
  if (hnan(a) || hnan(b)) return hfrom(0x7e00);
  if (a == (h16)0 && b == (h16)0) return hfrom((uint16_t)(hbits(a) | hbits(b)));
  return a < b ? a : b;
}

// The fp16 SiLU of the kernels (src/silu_lut.h:28-42): max(x, 0) - |x| q(|x|), q a piecewise quadratic in
// f = u - round(u) on 16 unit segments, u = min(|x|, 15.4). Coefficients as fp16 bit patterns: the values of
// src/silu_lut_tables_deg2.h. A NaN input gives NaN whichever segment it indexes.
static __constant__ uint16_t k_silu_c0[16] = {0x3800, 0x344e, 0x2fa1, 0x2a12, 0x249a, 0x1ed9, 0x1910, 0x1375,
                                              0x0d7e, 0x080a, 0x02f9, 0x0118, 0x0067, 0x0026, 0x000e, 0x0005};
static __constant__ uint16_t k_silu_c1[16] = {0xb40b, 0xb242, 0xaecc, 0xa9ea, 0xa4a6, 0x9f03, 0x9935, 0x93b1,
                                              0x8daa, 0x882c, 0x8312, 0x8121, 0x806a, 0x8027, 0x800e, 0x8005};
static __constant__ uint16_t k_silu_c2[16] = {0x23bd, 0x299d, 0x2915, 0x254c, 0x2073, 0x1ae1, 0x1528, 0x0fa3,
                                              0x09a2, 0x0426, 0x0187, 0x0090, 0x0035, 0x0013, 0x0007, 0x0003};
// the same with the three coefficient tables at c0, c1, c2 (LDS copies in the GEMM epilogue)
BNH_DEV h16 silu_lut_h_t(h16 x, const uint16_t *c0t, const uint16_t *c1t, const uint16_t *c2t) {
  const h16 magic = (h16)1536.0f;
  const h16 u = hfrom((uint16_t)(hbits(x) & 0x7fff));
  const h16 uc = hmin(u, hfrom(0x4bb3));  // (fp16)15.4f
  const h16 tm = uc + magic;
  const h16 f = uc - (tm - magic);
  unsigned n = hbits(tm) & 0xffu;
  if (n > 15) n = 0;
  const h16 c0 = hfrom(c0t[n]), c1 = hfrom(c1t[n]), c2 = hfrom(c2t[n]);
  h16 p = hfma(c2, f, c1);
  p = hfma(p, f, c0);
  return hfma(-u, p, hmax(x, (h16)0.0f));
}
BNH_DEV h16 silu_lut_h(h16 x) { return silu_lut_h_t(x, k_silu_c0, k_silu_c1, k_silu_c2); }

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// silu_lut_h on both halves of a packed pair, with the same roundings lane by lane: u = |x|; min(u, 15.4) (u is
// never NaN-sensitive here: a NaN x gives a NaN result through -u either way); the segment n in [0, 15] from the
// low byte of u + 1536; max(x, 0) as the sign-cleared x (FMAX(x, +0) for every non-NaN x, -0 included).
// t01[n] = c0 | c1 << 16, t2[n] = c2.
BNH_DEV h2 silu2_lut(h2 x, const uint32_t *t01, const uint16_t *t2) {
  const uint32_t xb = __builtin_bit_cast(uint32_t, x);
  const h2 u = __builtin_bit_cast(h2, xb & 0x7fff7fffu);
  const h2 uc = __builtin_elementwise_min(u, (h2){hfrom(0x4bb3), hfrom(0x4bb3)});
  const h2 magic = (h2){(h16)1536.0f, (h16)1536.0f};
  const h2 tm = uc + magic;
  const h2 f = uc - (tm - magic);
  const uint32_t tb = __builtin_bit_cast(uint32_t, tm);
  const uint32_t na = tb & 15u, nb = (tb >> 16) & 15u;
  const uint32_t ea = t01[na], eb = t01[nb];
  const h2 c0 = __builtin_bit_cast(h2, (ea & 0xffffu) | (eb << 16));
  const h2 c1 = __builtin_bit_cast(h2, (ea >> 16) | (eb & 0xffff0000u));
  const h2 c2 = __builtin_bit_cast(h2, (uint32_t)t2[na] | ((uint32_t)t2[nb] << 16));
  h2 p = __builtin_elementwise_fma(c2, f, c1);
  p = __builtin_elementwise_fma(p, f, c0);
  const uint32_t neg = ((xb >> 15) & 0x00010001u) * 0xffffu;  // all-ones halves where x is negative (or -0)
  const h2 m = __builtin_bit_cast(h2, xb & ~neg);
  return __builtin_elementwise_fma(-u, p, m);
}

#endif
