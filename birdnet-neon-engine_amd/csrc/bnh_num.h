// Device-side scalar numerics with the exact semantics of the AArch64 instructions libbnneon's NEON kernels use,
// so that every output element is bit-identical to the reference's (FPCR default: round to nearest even, denormals
// kept, FMIN/FMAX propagate NaN, float->int conversions saturate). All HIP sources are compiled with
// -ffp-contract=off: a*b+c is two roundings unless written as __builtin_fmaf.
#ifndef BNH_NUM_H
#define BNH_NUM_H
#include <hip/hip_runtime.h>
#include <stdint.h>

#define BNH_DEV __device__ __forceinline__

BNH_DEV uint32_t bnh_bits(float x) { return __float_as_uint(x); }
BNH_DEV float bnh_float(uint32_t u) { return __uint_as_float(u); }
BNH_DEV bool bnh_isnan(float x) { return x != x; }

// FMAX / FMIN (NEON vmaxq_f32 / vminq_f32): a NaN operand gives a NaN; +0 orders above -0
BNH_DEV float bnh_fmax(float a, float b) {
  if (bnh_isnan(a)) return bnh_float(bnh_bits(a) | 0x400000u);
  if (bnh_isnan(b)) return bnh_float(bnh_bits(b) | 0x400000u);
  if (a == 0.f && b == 0.f) return bnh_float(bnh_bits(a) & bnh_bits(b));
  return a > b ? a : b;
}
BNH_DEV float bnh_fmin(float a, float b) {
  if (bnh_isnan(a)) return bnh_float(bnh_bits(a) | 0x400000u);
  if (bnh_isnan(b)) return bnh_float(bnh_bits(b) | 0x400000u);
  if (a == 0.f && b == 0.f) return bnh_float(bnh_bits(a) | bnh_bits(b));
  return a < b ? a : b;
}
// FMAXNM / FMINNM (C fmaxf / fminf on AArch64): a NaN operand is ignored
BNH_DEV float bnh_fmaxnm(float a, float b) {
  if (bnh_isnan(a)) return b;
  if (bnh_isnan(b)) return a;
  return bnh_fmax(a, b);
}
BNH_DEV float bnh_fminnm(float a, float b) {
  if (bnh_isnan(a)) return b;
  if (bnh_isnan(b)) return a;
  return bnh_fmin(a, b);
}

BNH_DEV int32_t bnh_sat_s32(float r) {  // r integral, or NaN / inf
  if (bnh_isnan(r)) return 0;
  if (r >= 2147483648.f) return INT32_MAX;
  if (r < -2147483648.f) return INT32_MIN;
  return (int32_t)r;
}
// FCVTNS (vcvtnq_s32_f32): nearest even, int32-saturating
BNH_DEV int32_t bnh_cvtn_s32(float x) { return bnh_sat_s32(__builtin_rintf(x)); }
// FCVTZS w (the C cast float -> int32 on AArch64): toward zero, saturating, NaN -> 0
BNH_DEV int32_t bnh_cvtz_s32(float x) { return bnh_sat_s32(__builtin_truncf(x)); }
// FCVTAS (vcvtaq_s32_f32): nearest, ties away from zero, int32-saturating
BNH_DEV int32_t bnh_cvta_s32(float x) {
  float t = __builtin_truncf(x);
  float d = x - t;  // exact
  if (d >= 0.5f) t += 1.f;
  else if (d <= -0.5f) t -= 1.f;
  return bnh_sat_s32(t);
}
// (int32_t)lrintf(x) on AArch64: FRINTX, FCVTZS to 64 bits (saturating), low 32 bits kept
BNH_DEV int32_t bnh_lrintf_s32(float x) {
  float r = __builtin_rintf(x);
  if (bnh_isnan(r)) return 0;
  if (r >= 9223372036854775808.f) return -1;          // INT64_MAX, low word
  if (r < -9223372036854775808.f) return 0;           // INT64_MIN, low word
  if (r >= 2147483648.f || r < -2147483648.f) return (int32_t)(uint32_t)(uint64_t)(int64_t)r;
  return (int32_t)r;
}

// FRECPE for binary32 (Arm ARM FPRecipEstimate, FZ = 0, round to nearest). The 9-bit estimate
// r = (floor(2^19 / (2a + 1)) + 1) / 2 is computed as floor(2^19 * rcp(2a + 1)): for 2a + 1 in [513, 1023] the
// quotient is at least 1/1023 away from an integer on either side and the approximate reciprocal is off by less
// than 3e-4 absolute, so the floor is exact.
BNH_DEV int bnh_recip_estimate(int a) {
  int d = 2 * a + 1;
  int b = (int)__builtin_floorf(524288.f * __builtin_amdgcn_rcpf((float)d));
  return (b + 1) >> 1;
}
BNH_DEV float bnh_frecpe(float x) {
  uint32_t u = bnh_bits(x), sign = u & 0x80000000u, ex = (u >> 23) & 0xffu, fr = u & 0x7fffffu;
  if (ex == 0xffu) return fr ? bnh_float(u | 0x400000u) : bnh_float(sign);
  if (ex == 0 && fr < 0x200000u) return bnh_float(sign | 0x7f800000u);  // zero, or below 2^-128: overflow
  int e = (int)ex;
  uint32_t f23 = fr;
  if (e == 0) {  // denormal: normalise by one or two places
    if (!(f23 & 0x400000u)) { e = -1; f23 = (f23 << 2) & 0x7fffffu; }
    else f23 = (f23 << 1) & 0x7fffffu;
  }
  int est = bnh_recip_estimate(256 | (int)(f23 >> 15));
  int rexp = 253 - e;
  uint32_t rf = (uint32_t)(est & 0xff) << 15;
  if (rexp == 0) rf = 0x400000u | (rf >> 1);
  else if (rexp == -1) { rf = 0x200000u | (rf >> 2); rexp = 0; }
  return bnh_float(sign | ((uint32_t)(rexp & 0xff) << 23) | rf);
}
// FRECPS: 2 - a*b with one rounding; (inf, 0) -> 2
BNH_DEV float bnh_frecps(float a, float b) {
  if (bnh_isnan(a)) return bnh_float(bnh_bits(a) | 0x400000u);
  if (bnh_isnan(b)) return bnh_float(bnh_bits(b) | 0x400000u);
  bool ia = __builtin_isinf(a), ib = __builtin_isinf(b);
  if ((ia && b == 0.f) || (a == 0.f && ib)) return 2.f;
  if (ia || ib) return ((bnh_bits(a) ^ bnh_bits(b)) & 0x80000000u) ? __builtin_inff() : -__builtin_inff();
  return __builtin_fmaf(-a, b, 2.f);
}

// The fp32 SiLU of libbnneon's GEMM / depthwise epilogues (src/gemm_f32.h:102-118): exp2 by the magic-number split
// and a degree-5 polynomial, t clamped to +-60, one FRECPE + FRECPS Newton step. Because of the clamp, the divisor
// d = 1 + 2^t lies in [1, 2^60 + 1] (finite, normal, positive) for every x that is not NaN, so FRECPE reduces to its
// normal-operand case (exponent 253 - e, 8 fraction bits from the 9-bit estimate of the leading 8 significand bits)
// and FRECPS to one fused 2 - d r. A NaN x gives NaN through the final product x r whatever the clamp did with it
// (the reference's NaN travels through d and r instead: the same NaN result, payloads aside).
// Per leading significand byte of d: 253 << 23 with the estimate's fraction bits at 22..15. bnh_silu_f32_t subtracts
// d's exponent field from it, giving FRECPE's exponent 253 - e over the same fraction (no borrow reaches the fraction:
// e <= 127 + 61). A block puts this table in LDS (bnh_silu_table, then a barrier) for bnh_silu_f32_t.
BNH_DEV void bnh_silu_table(uint32_t *tbl) {
  for (int i = threadIdx.x; i < 256; i += blockDim.x)
    tbl[i] = 253u << 23 | (uint32_t)(bnh_recip_estimate(256 | i) & 0xff) << 15;
}
BNH_DEV float bnh_silu_d(float x) {  // the divisor d = 1 + 2^t, t = clamp(-x log2 e, -60, 60)
  const float magic = 12582912.0f;
  float t = x * -1.44269504f;
  t = __builtin_amdgcn_fmed3f(t, -60.f, 60.f);
  const float tm = t + magic;
  const float f = t - (tm - magic);
  const uint32_t ni = bnh_bits(tm) << 23;
  float p = __builtin_fmaf(1.3333558e-3f, f, 9.6181291e-3f);
  p = __builtin_fmaf(p, f, 5.5504109e-2f);
  p = __builtin_fmaf(p, f, 2.4022651e-1f);
  p = __builtin_fmaf(p, f, 6.9314718e-1f);
  p = __builtin_fmaf(p, f, 1.0f);
  return 1.f + bnh_float(bnh_bits(p) + ni);
}
BNH_DEV float bnh_silu_f32_t(float x, const uint32_t *tbl) {
  const float d = bnh_silu_d(x);
  const uint32_t db = bnh_bits(d);
  float r = bnh_float(tbl[(db >> 15) & 0xffu] - (db & 0x7f800000u));
  r = r * __builtin_fmaf(-d, r, 2.f);
  return x * r;
}
BNH_DEV float bnh_silu_f32(float x) {  // the same without the table
  const float d = bnh_silu_d(x);
  const uint32_t db = bnh_bits(d);
  const int est = bnh_recip_estimate(256 | (int)((db >> 15) & 0xffu));
  float r = bnh_float(((253u << 23) - (db & 0x7f800000u)) | ((uint32_t)(est & 0xff) << 15));
  r = r * __builtin_fmaf(-d, r, 2.f);
  return x * r;
}
// n / d for 0 <= n < 2^52 and 1 <= d < 2^31, given rd = 1.0 / d: the double product is within 2^-21 of n / d, so
// its truncation is off by at most one, which one remainder test corrects
BNH_DEV int bnh_div(long long n, int d, double rd) {
  int q = (int)((double)n * rd);
  const long long r = n - (long long)q * d;
  if (r < 0) q--;
  else if (r >= d) q++;
  return q;
}
// The logical index of hardware block b of a 1-D grid of n blocks. The hardware places block b on XCD b % 8; this
// gives the blocks of one XCD one contiguous range of logical indices, so that work on neighbouring data (the rows a
// stencil shares) runs under one XCD's L2.
BNH_DEV unsigned bnh_xcd_block(unsigned b, unsigned n) {
  const unsigned q = n / 8, r = n % 8, x = b % 8;
  return x * q + (x < r ? x : r) + b / 8;
}
// ReLU as vmaxq_f32(y, 0): -0 -> +0, NaN stays NaN
BNH_DEV float bnh_relu_f32(float y) { return bnh_fmax(y, 0.f); }

// gemmlowp fixed point (the Q31 requant specification of the int8 GEMM / depthwise of this library, shift 0..31),
// in 32-bit forms around one 64-bit multiply-add, with no branches:
//  * SaturatingRoundingDoublingHighMul(a, b) = (a b + nudge) / 2^31 truncated, nudge = 2^30 for a b >= 0 and
//    1 - 2^30 below; both cases equal floor((a b + 2^30) / 2^31) (for a b < 0 the truncation of n = a b + 1 - 2^30 is
//    floor((n + 2^31 - 1) / 2^31)). That floor lies in [-2^31 + 1, 2^31] and reaches 2^31, whose low 32 bits read
//    INT32_MIN, only for INT32_MIN x INT32_MIN: the one overflow, which saturates to INT32_MAX.
//  * RoundingDivideByPOT(x, e) (round half away from zero) = (x >> e) + [(x & mask) > (mask >> 1) + [x < 0]],
//    mask = 2^e - 1 (for e = 0 the mask is 0 and x is returned).
BNH_DEV int32_t bnh_requant(int32_t acc, int32_t mult, int shift, int zy, int lo, int hi) {
  int32_t r = (int32_t)(uint32_t)((uint64_t)((int64_t)acc * mult + (1LL << 30)) >> 31);
  r = r == INT32_MIN ? INT32_MAX : r;
  const int32_t mask = (int32_t)((1u << shift) - 1u);
  const int32_t v = (r >> shift) + ((r & mask) > (mask >> 1) + (int32_t)((uint32_t)r >> 31) ? 1 : 0);
  // clamp(v + zy (saturating), lo, hi) for lo <= hi: the median of the three, one v_med3_i32
  int32_t y;
  asm("v_med3_i32 %0, %1, %2, %3" : "=v"(y) : "v"(__builtin_elementwise_add_sat(v, zy)), "v"(lo), "v"(hi));
  return y;
}
// The same for shift e in 1..31 as one rounding of the 64-bit product: floor((floor(p / 2^31) + c) / 2^e) =
// floor((p + c 2^31) / 2^(31 + e)) for integer c, so with c = 2^(e-1) - [p < 0] and p = acc m + 2^30
//   RDBYPOT(SRDHM(acc, m), e) = floor((acc m + 2^30 + 2^(30+e) - [p < 0] 2^31) / 2^(31+e)),
// the high word of one 64-bit multiply-add shifted right by e - 1. [p < 0] may be read from the operands' signs:
// where they disagree (acc m in [-2^30, 0), or a zero product with a negative operand) SRDHM is 0 and so is the
// result either way. INT32_MIN x INT32_MIN gives 2^(31-e), the value of the saturated SRDHM, by itself. The two
// addends per shift are taken out of the loop by the caller (BnhRqS1).
struct BnhRqS1 {
  int64_t a0, a1;  // 2^30 + 2^(30+e), and that minus 2^31
  int e1;          // e - 1
};
BNH_DEV BnhRqS1 bnh_rq_s1(int shift) {
  BnhRqS1 c;
  c.a0 = (1LL << 30) + (1LL << (30 + shift));
  c.a1 = c.a0 - (1LL << 31);
  c.e1 = shift - 1;
  return c;
}
BNH_DEV int32_t bnh_requant_s1(int32_t acc, int32_t mult, BnhRqS1 c, int zy, int lo, int hi) {
  const int64_t q = (int64_t)acc * mult + ((acc ^ mult) < 0 ? c.a1 : c.a0);
  const int32_t v = (int32_t)(q >> 32) >> c.e1;
  int32_t y;
  asm("v_med3_i32 %0, %1, %2, %3" : "=v"(y) : "v"(__builtin_elementwise_add_sat(v, zy)), "v"(lo), "v"(hi));
  return y;
}
// 4 x 4 byte transpose: r_i holds bytes (i, 0..3); c_j receives bytes (0..3, j)
BNH_DEV void transpose4x4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3, uint32_t c[4]) {
  // r_i = bytes of k row i for pixels 0..3; c_j = bytes of pixel j for k rows 0..3
  const uint32_t a_lo = __builtin_amdgcn_perm(r1, r0, 0x05010400u), a_hi = __builtin_amdgcn_perm(r1, r0, 0x07030602u);
  const uint32_t b_lo = __builtin_amdgcn_perm(r3, r2, 0x05010400u), b_hi = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
  c[0] = __builtin_amdgcn_perm(b_lo, a_lo, 0x05040100u);
  c[1] = __builtin_amdgcn_perm(b_lo, a_lo, 0x07060302u);
  c[2] = __builtin_amdgcn_perm(b_hi, a_hi, 0x05040100u);
  c[3] = __builtin_amdgcn_perm(b_hi, a_hi, 0x07060302u);
}
#endif
