/* CPU oracle (test infrastructure only): libbnneon's depthwise convolutions (fp32 DWK / DW3, fp16 DWK / DW3), the
 * exact fp16 arithmetic they run in, the fp16 LUT SiLU, and this project's int8 depthwise specification. See
 * oracle.h. fp16 values are carried as their bit patterns (uint16_t); every fp16 operation is computed exactly and
 * rounded once to nearest even, with fp16 denormals, as the AArch64 fp16 instructions do (FPCR.FZ16 = 0). */
#include <math.h>
#include <string.h>

#include "oracle.h"

/* ---------------------------------------------------------------- fp16 arithmetic */
static int h_isnan(uint16_t h) { return (h & 0x7c00) == 0x7c00 && (h & 0x3ff); }
static int h_isinf(uint16_t h) { return (h & 0x7fff) == 0x7c00; }

float orc_h2f(uint16_t h) {
  int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(1024 + m), e - 25);
  return s ? -v : v;
}

/* round sign * S * 2^e0 (S > 0, exact) to fp16, nearest even */
static uint16_t h_round(int sign, unsigned __int128 S, int e0) {
  int L = 0;
  for (unsigned __int128 t = S; t; t >>= 1) L++;
  int er = e0 + L - 11;            /* exponent of the result's last mantissa bit */
  if (er < -24) er = -24;          /* denormal range: last bit fixed at 2^-24 */
  unsigned __int128 M;
  int sh = er - e0;
  if (sh > 0) {
    unsigned __int128 q = S >> sh, r = S & ((((unsigned __int128)1) << sh) - 1), half = ((unsigned __int128)1) << (sh - 1);
    if (r > half || (r == half && (q & 1))) q++;
    M = q;
  } else
    M = S << (-sh);
  if (M >= 2048) { M >>= 1; er++; }  /* rounding carried into a new bit (M was 2047 + 1 -> 2048, exact shift) */
  uint16_t out;
  if (M < 1024) out = (uint16_t)M;   /* denormal (er == -24) */
  else {
    int ef = er + 25;                /* biased exponent of M * 2^er with M in [1024, 2048) */
    if (ef >= 31) out = 0x7c00;      /* overflow: infinity */
    else out = (uint16_t)((ef << 10) | ((int)M - 1024));
  }
  return (uint16_t)(out | (sign ? 0x8000 : 0));
}

/* a * b + c with one rounding (FMLA / vfmaq_f16) */
uint16_t orc_h_fma(uint16_t a, uint16_t b, uint16_t c) {
  if (h_isnan(a) || h_isnan(b) || h_isnan(c)) return 0x7e00;
  int sp = (a ^ b) >> 15, sc = c >> 15;
  int pz = !(a & 0x7fff) || !(b & 0x7fff);
  if (h_isinf(a) || h_isinf(b)) {
    if (pz) return 0x7e00;                               /* inf * 0 */
    if (h_isinf(c) && sc != sp) return 0x7e00;           /* inf - inf */
    return (uint16_t)(0x7c00 | (sp << 15));
  }
  if (h_isinf(c)) return c;
  int ea = (a >> 10) & 31, eb = (b >> 10) & 31, ec = (c >> 10) & 31;
  unsigned Ma = ea ? 1024 + (a & 1023) : (a & 1023), Mb = eb ? 1024 + (b & 1023) : (b & 1023);
  unsigned Mc = ec ? 1024 + (c & 1023) : (c & 1023);
  int Ea = ea ? ea - 25 : -24, Eb = eb ? eb - 25 : -24, Ec = ec ? ec - 25 : -24;
  unsigned __int128 P = (unsigned __int128)Ma * Mb, Cm = Mc;
  int Ep = Ea + Eb;
  if (P == 0 && Cm == 0) return (uint16_t)((sp && sc) ? 0x8000 : 0);  /* exact zero: +0 unless both -0 */
  int e0 = Ep < Ec ? Ep : Ec;
  P <<= (Ep - e0);
  Cm <<= (Ec - e0);
  if (sp == sc) return h_round(sp, P + Cm, e0);
  if (P == Cm) return 0;                                   /* x - x = +0 */
  if (P > Cm) return h_round(sp, P - Cm, e0);
  return h_round(sc, Cm - P, e0);
}
uint16_t orc_h_add(uint16_t a, uint16_t b) { return orc_h_fma(a, 0x3c00, b); }
uint16_t orc_h_mul(uint16_t a, uint16_t b) { return orc_h_fma(a, b, 0x8000); }

/* FMAX / FMIN on fp16 */
uint16_t orc_h_max(uint16_t a, uint16_t b) {
  if (h_isnan(a) || h_isnan(b)) return 0x7e00;
  float x = orc_h2f(a), y = orc_h2f(b);
  if (x == 0 && y == 0) return (uint16_t)(a & b & 0x8000);
  return x > y ? a : b;
}
uint16_t orc_h_min(uint16_t a, uint16_t b) {
  if (h_isnan(a) || h_isnan(b)) return 0x7e00;
  float x = orc_h2f(a), y = orc_h2f(b);
  if (x == 0 && y == 0) return (uint16_t)((a | b) & 0x8000);
  return x < y ? a : b;
}

/* The fp16 SiLU of libbnneon's kernels (src/silu_lut.h:28-42): silu(x) = max(x, 0) - |x| q(|x|), q(u) ~ sigmoid(-u)
 * by a 16-segment piecewise quadratic in f = u - round(u), u clamped to 15.4, coefficients fp16. The coefficient
 * values are those of src/silu_lut_tables_deg2.h (c0[n], c1[n], c2[n] for n = round(u)), as fp16 bit patterns. */
static const uint16_t SILU_C0[16] = {0x3800, 0x344e, 0x2fa1, 0x2a12, 0x249a, 0x1ed9, 0x1910, 0x1375,
                                     0x0d7e, 0x080a, 0x02f9, 0x0118, 0x0067, 0x0026, 0x000e, 0x0005};
static const uint16_t SILU_C1[16] = {0xb40b, 0xb242, 0xaecc, 0xa9ea, 0xa4a6, 0x9f03, 0x9935, 0x93b1,
                                     0x8daa, 0x882c, 0x8312, 0x8121, 0x806a, 0x8027, 0x800e, 0x8005};
static const uint16_t SILU_C2[16] = {0x23bd, 0x299d, 0x2915, 0x254c, 0x2073, 0x1ae1, 0x1528, 0x0fa3,
                                     0x09a2, 0x0426, 0x0187, 0x0090, 0x0035, 0x0013, 0x0007, 0x0003};
/* a TBL of the 32-byte table (low bytes, then high bytes) at byte indices n (low) and n + 16 (high): 0 past 32 */
static uint16_t lut_coef(const uint16_t *c, unsigned n) {
  unsigned lo = n < 16 ? (c[n] & 0xff) : (n < 32 ? (c[n - 16] >> 8) : 0);
  unsigned n2 = (n + 16) & 0xff;
  unsigned hi = n2 < 16 ? (c[n2] & 0xff) : (n2 < 32 ? (c[n2 - 16] >> 8) : 0);
  return (uint16_t)(lo | (hi << 8));
}
uint16_t orc_silu_lut_h(uint16_t x) {
  const uint16_t magic = 0x6600, umax = 0x4bb3; /* 1536.0, (fp16)15.4f = 15.3984375 */
  uint16_t u = (uint16_t)(x & 0x7fff);
  uint16_t uc = orc_h_min(u, umax);
  uint16_t tm = orc_h_add(uc, magic);
  uint16_t f = orc_h_add(uc, (uint16_t)(orc_h_add(tm, 0xe600 /* -1536 */) ^ 0x8000));
  unsigned n = tm & 0xff;
  uint16_t c0 = lut_coef(SILU_C0, n), c1 = lut_coef(SILU_C1, n), c2 = lut_coef(SILU_C2, n);
  uint16_t p = orc_h_fma(c2, f, c1);
  p = orc_h_fma(p, f, c0);
  return orc_h_fma((uint16_t)(u ^ 0x8000), p, orc_h_max(x, 0));
}

/* ---------------------------------------------------------------- fp32 DWK (src/pc_kern_f32.c:163-334) */
/* out [Ho][Wo][C], xp zero-haloed by h = (k-1)/2, w [k*k][C]. Per output: the first Wo & ~3 pixels of a row run two
 * fused chains (bias + even taps, 0 + odd taps, tap order (ky, kx)) then one add; the last Wo % 4 one chain from the
 * bias. chsum[c]: per row, each 4-pixel group adds (v0 + v1) + (v2 + v3), each tail pixel its value, in order. */
void orc_dwk_f32(const float *xp, int H, int W, int C, int k, int s, int pt, int pl, const float *w, const float *b,
                 int act, float *out, int Ho, int Wo, float *chsum) {
  (void)H;
  const int h = (k - 1) / 2, Wp = W + 2 * h;
  for (int c = 0; c < C; c++) chsum[c] = 0.f;
  for (int oy = 0; oy < Ho; oy++) {
    const int g4 = Wo & ~3;
    for (int ox = 0; ox < Wo; ox++)
      for (int c = 0; c < C; c++) {
        const float *x0 = xp + ((size_t)(oy * s - pt + h) * Wp + (ox * s - pl + h)) * C + c;
        float a = b[c], e = 0.f;
        for (int t = 0; t < k * k; t++) {
          float xv = x0[((size_t)(t / k) * Wp + t % k) * C], wv = w[(size_t)t * C + c];
          if (ox < g4 && (t & 1)) e = fmaf(xv, wv, e);
          else a = fmaf(xv, wv, a);
        }
        float v = ox < g4 ? a + e : a;
        if (act == 1) v = orc_silu_f32(v);
        out[((size_t)oy * Wo + ox) * C + c] = v;
      }
    for (int c = 0; c < C; c++) {
      const float *o = out + (size_t)oy * Wo * C + c;
      for (int ox = 0; ox < g4; ox += 4)
        chsum[c] = chsum[c] + ((o[(size_t)ox * C] + o[(size_t)(ox + 1) * C]) + (o[(size_t)(ox + 2) * C] + o[(size_t)(ox + 3) * C]));
      for (int ox = g4; ox < Wo; ox++) chsum[c] = chsum[c] + o[(size_t)ox * C];
    }
  }
}

/* ---------------------------------------------------------------- fp32 DW3 (src/gemm_f32.c:213-441) */
/* 3x3, halo 1, rows oy*s.., columns ox*s..: three partial sums by tap column (the first two start with a multiply),
 * acc = bias-chain + (col1 + col2); SiLU always; chsum = the outputs added pixel by pixel in raster order */
void orc_dw3_f32(const float *xp, int H, int W, int C, int s, const float *w, const float *b, float *out, int Ho,
                 int Wo, float *chsum) {
  (void)H;
  const int Wp = W + 2;
  for (int c = 0; c < C; c++) chsum[c] = 0.f;
  for (int oy = 0; oy < Ho; oy++)
    for (int ox = 0; ox < Wo; ox++)
      for (int c = 0; c < C; c++) {
        const float *q = xp + ((size_t)(oy * s) * Wp + ox * s) * C + c;
        const size_t r1 = (size_t)Wp * C, r2 = 2 * r1;
#define X(row, col) q[(row) + (size_t)(col) * C]
#define WT(t) w[(size_t)(t) * C + c]
        float acc = fmaf(WT(0), X(0, 0), b[c]);
        float acb = WT(1) * X(0, 1);
        float acd = WT(2) * X(0, 2);
        acc = fmaf(WT(3), X(r1, 0), acc);
        acb = fmaf(WT(4), X(r1, 1), acb);
        acd = fmaf(WT(5), X(r1, 2), acd);
        acc = fmaf(WT(6), X(r2, 0), acc);
        acb = fmaf(WT(7), X(r2, 1), acb);
        acd = fmaf(WT(8), X(r2, 2), acd);
#undef X
#undef WT
        float v = orc_silu_f32(acc + (acb + acd));
        out[((size_t)oy * Wo + ox) * C + c] = v;
        chsum[c] = chsum[c] + v;
      }
}

/* ---------------------------------------------------------------- fp16 DWK (src/pc_kern_f16.c:16-96) */
/* fp16 chains from the fp16 bias: 4-pixel groups split even / odd taps, then a 2-pixel and a 1-pixel tail with one
 * chain each; LUT SiLU; chsum in fp32 from per-group fp16 sums ((v0+v1)+(v2+v3), v0+v1, v0) */
void orc_dwk_f16(const uint16_t *xp, int H, int W, int C, int k, int s, int pt, int pl, const uint16_t *w,
                 const uint16_t *b, int act, uint16_t *out, int Ho, int Wo, float *chsum) {
  (void)H;
  const int h = (k - 1) / 2, Wp = W + 2 * h;
  const int g4 = Wo & ~3, g2 = g4 + ((Wo - g4) & 2);
  for (int c = 0; c < C; c++) chsum[c] = 0.f;
  for (int oy = 0; oy < Ho; oy++) {
    for (int ox = 0; ox < Wo; ox++)
      for (int c = 0; c < C; c++) {
        const uint16_t *x0 = xp + ((size_t)(oy * s - pt + h) * Wp + (ox * s - pl + h)) * C + c;
        uint16_t a = b[c], e = 0;
        for (int t = 0; t < k * k; t++) {
          uint16_t xv = x0[((size_t)(t / k) * Wp + t % k) * C], wv = w[(size_t)t * C + c];
          if (ox < g4 && (t & 1)) e = orc_h_fma(xv, wv, e);
          else a = orc_h_fma(xv, wv, a);
        }
        uint16_t v = ox < g4 ? orc_h_add(a, e) : a;
        if (act == 1) v = orc_silu_lut_h(v);
        out[((size_t)oy * Wo + ox) * C + c] = v;
      }
    for (int c = 0; c < C; c++) {
      const uint16_t *o = out + (size_t)oy * Wo * C + c;
#define O(i) o[(size_t)(i) * C]
      for (int ox = 0; ox < g4; ox += 4)
        chsum[c] = chsum[c] + orc_h2f(orc_h_add(orc_h_add(O(ox), O(ox + 1)), orc_h_add(O(ox + 2), O(ox + 3))));
      if (g2 > g4) chsum[c] = chsum[c] + orc_h2f(orc_h_add(O(g4), O(g4 + 1)));
      if (Wo > g2) chsum[c] = chsum[c] + orc_h2f(O(g2));
#undef O
    }
  }
}

/* ---------------------------------------------------------------- fp16 DW3 (src/kern_f16.c:83-155) */
/* 3x3 on a halo-1 input at rows oy*s - pt + 1, columns ox*s - pl + 1: two fp16 chains (bias-FMA and a first
 * multiply) interleaved over the taps, their sum, the LUT SiLU always; per row an fp16 running sum of the outputs in
 * order, added to the fp32 chsum at the row's end */
void orc_dw3_f16(const uint16_t *xp, int H, int W, int C, int s, int pt, int pl, const uint16_t *w, const uint16_t *b,
                 uint16_t *out, int Ho, int Wo, float *chsum) {
  (void)H;
  const int Wp = W + 2;
  for (int c = 0; c < C; c++) chsum[c] = 0.f;
  for (int oy = 0; oy < Ho; oy++) {
    const int iy0 = oy * s - pt + 1;
    for (int c = 0; c < C; c++) {
      uint16_t rs = 0;
      for (int ox = 0; ox < Wo; ox++) {
        const int ix0 = ox * s - pl + 1;
        const uint16_t *r0 = xp + ((size_t)iy0 * Wp + ix0) * C + c, *r1 = r0 + (size_t)Wp * C, *r2 = r1 + (size_t)Wp * C;
#define WT(t) w[(size_t)(t) * C + c]
        uint16_t a = orc_h_fma(r0[0], WT(0), b[c]);
        uint16_t a2 = orc_h_mul(r0[C], WT(1));
        a = orc_h_fma(r0[2 * C], WT(2), a);
        a2 = orc_h_fma(r1[0], WT(3), a2);
        a = orc_h_fma(r1[C], WT(4), a);
        a2 = orc_h_fma(r1[2 * C], WT(5), a2);
        a = orc_h_fma(r2[0], WT(6), a);
        a2 = orc_h_fma(r2[C], WT(7), a2);
        a = orc_h_fma(r2[2 * C], WT(8), a);
#undef WT
        uint16_t y = orc_silu_lut_h(orc_h_add(a, a2));
        out[((size_t)oy * Wo + ox) * C + c] = y;
        rs = orc_h_add(rs, y);
      }
      chsum[c] = chsum[c] + orc_h2f(rs);
    }
  }
}

/* ---------------------------------------------------------------- int8 depthwise (own specification) */
/* x int8 [H][W][C] with zero point zx, 'same'-style padding by pt / pl (taps outside the image contribute nothing,
 * as a zero-point pad would), w int8 [k*k][C] symmetric per channel, bias int32 [C]:
 *   acc = bias[c] + sum over in-image taps of w[t][c] * (x - zx)          (int32)
 *   y = clamp(RoundingDivideByPOT(SRDHM(acc, mult[c]), shift[c]) + zy, lo, hi)
 *   out = lut ? lut[y + 128] : y                                           (the SiLU as an int8 -> int8 table) */
void orc_dw_s8(const int8_t *x, int H, int W, int C, int k, int s, int pt, int pl, const int8_t *w, const int32_t *bias,
               const int32_t *mult, const int32_t *shift, int zx, int zy, int lo, int hi, const int8_t *lut, int8_t *out,
               int Ho, int Wo) {
  for (int oy = 0; oy < Ho; oy++)
    for (int ox = 0; ox < Wo; ox++)
      for (int c = 0; c < C; c++) {
        uint32_t acc = (uint32_t)bias[c];
        for (int ky = 0; ky < k; ky++)
          for (int kx = 0; kx < k; kx++) {
            int iy = oy * s - pt + ky, ix = ox * s - pl + kx;
            if (iy < 0 || iy >= H || ix < 0 || ix >= W) continue;
            acc += (uint32_t)((int32_t)w[(size_t)(ky * k + kx) * C + c] * ((int32_t)x[((size_t)iy * W + ix) * C + c] - zx));
          }
        int8_t y = orc_requant((int32_t)acc, mult[c], shift[c], zy, lo, hi);
        out[((size_t)oy * Wo + ox) * C + c] = lut ? lut[(int)y + 128] : y;
      }
}
