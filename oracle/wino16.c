/* CPU oracle (test infrastructure only): libbnneon's fp16 Winograd F(2x2,3x3) for 24 channels (src/wino_s0.c:1-165,
 * the CONV3C24 op of src/rt_ops_dot.c:63-107) and the fp16 reciprocal estimate / step it uses. See oracle.h. fp16
 * values are bit patterns; arithmetic through orc_h_* (dw.c), one rounding per operation. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static int h_nan(uint16_t h) { return (h & 0x7c00) == 0x7c00 && (h & 0x3ff); }

/* FRECPE, half precision (Arm ARM FPRecipEstimate with N = 16, FPCR.FZ16 = 0, round to nearest) */
uint16_t orc_frecpe_h(uint16_t x) {
  const uint16_t sign = x & 0x8000u, exp = (x >> 10) & 31u, frac = x & 0x3ffu;
  if (exp == 31 && frac) return (uint16_t)(x | 0x200u);            /* NaN: quieted operand */
  if (exp == 31) return sign;                                       /* +-inf -> +-0 */
  if (exp == 0 && frac == 0) return (uint16_t)(sign | 0x7c00u);     /* +-0 -> +-inf */
  if (exp == 0 && frac < 0x100u) return (uint16_t)(sign | 0x7c00u); /* |x| < 2^-16: overflow, RN -> inf */
  uint64_t fraction = (uint64_t)frac << 42;                         /* 52-bit fraction field */
  int e = (int)exp;
  if (e == 0) {
    if (!((fraction >> 51) & 1)) { e = -1; fraction = (fraction & ((1ull << 50) - 1)) << 2; }
    else fraction = (fraction & ((1ull << 51) - 1)) << 1;
  }
  const int scaled = 256 | (int)((fraction >> 44) & 0xffu);
  int result_exp = 29 - e;
  const int est = orc_recip_estimate(scaled);
  fraction = (uint64_t)(est & 0xff) << 44;
  if (result_exp == 0) fraction = (1ull << 51) | (fraction >> 1);
  else if (result_exp == -1) { fraction = (1ull << 50) | (fraction >> 2); result_exp = 0; }
  return (uint16_t)(sign | ((unsigned)(result_exp & 31) << 10) | (unsigned)((fraction >> 42) & 0x3ffu));
}

/* FRECPS, half precision: 2 - a*b with one rounding; (inf, 0) and (0, inf) give +2 */
uint16_t orc_frecps_h(uint16_t a, uint16_t b) {
  if (h_nan(a)) return (uint16_t)(a | 0x200u);
  if (h_nan(b)) return (uint16_t)(b | 0x200u);
  const int ainf = (a & 0x7fff) == 0x7c00, binf = (b & 0x7fff) == 0x7c00;
  const int az = !(a & 0x7fff), bz = !(b & 0x7fff);
  if ((ainf && bz) || (az && binf)) return 0x4000;                  /* 2.0 */
  return orc_h_fma((uint16_t)(a ^ 0x8000u), b, 0x4000);
}

/* silu4w (src/wino_s0.c:14-34): the polynomial fp16 SiLU of act.h's silu_f16_a */
uint16_t orc_silu_poly_h(uint16_t x) {
  const uint16_t k = orc_f2h(-1.44269504f), lo = orc_f2h(-14.f), hi = orc_f2h(14.f), magic = orc_f2h(1536.0f);
  const uint16_t c3 = orc_f2h(0.0555041f), c2 = orc_f2h(0.2402265f), c1 = orc_f2h(0.6931472f), one = 0x3c00;
  const uint16_t t = orc_h_min(orc_h_max(orc_h_mul(x, k), lo), hi);
  const uint16_t tm = orc_h_add(t, magic);
  const uint16_t f = orc_h_add(t, (uint16_t)(orc_h_add(tm, (uint16_t)(magic ^ 0x8000u)) ^ 0x8000u));
  uint16_t pp = orc_h_fma(c3, f, c2);
  pp = orc_h_fma(pp, f, c1);
  pp = orc_h_fma(pp, f, one);
  const uint16_t d = orc_h_add((uint16_t)(pp + (uint16_t)(tm << 10)), one);
  uint16_t r = orc_frecpe_h(d);
  r = orc_h_mul(r, orc_frecps_h(d, r));
  return orc_h_mul(x, r);
}

static const float G[4][3] = {{1, 0, 0}, {.5f, .5f, .5f}, {.5f, -.5f, .5f}, {0, 0, 1}};

/* wino_s0_pack (src/wino_s0.c:40-64): U fp16 [16][24 ci][24 co], bias fp16 [24] */
void orc_wino_s0_pack(const float *w, const float *bias, uint16_t *U, uint16_t *b16) {
  for (int co = 0; co < 24; co++) {
    b16[co] = orc_f2h(bias[co]);
    for (int ci = 0; ci < 24; ci++) {
      float g[3][3], t[4][3], u[4][4];
      for (int ky = 0; ky < 3; ky++)
        for (int kx = 0; kx < 3; kx++) g[ky][kx] = w[((co * 3 + ky) * 3 + kx) * 24 + ci];
      for (int i = 0; i < 4; i++)
        for (int kx = 0; kx < 3; kx++) t[i][kx] = G[i][0] * g[0][kx] + G[i][1] * g[1][kx] + G[i][2] * g[2][kx];
      for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) u[i][j] = t[i][0] * G[j][0] + t[i][1] * G[j][1] + t[i][2] * G[j][2];
      for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) U[((size_t)(i * 4 + j) * 24 + ci) * 24 + co] = orc_f2h(u[i][j]);
    }
  }
}

#define HADD orc_h_add
#define HSUB(a, b) orc_h_add((a), (uint16_t)((b) ^ 0x8000u))

/* conv3x3_s1_wino_f16_c24_rows over every tile row (src/wino_s0.c:145-165): x, out padded [H+2][W+2][24] fp16, the
 * residual is x itself; out's halo is left as the caller set it */
void orc_wino_s0(const uint16_t *x, int H, int W, const uint16_t *U, const uint16_t *b16, uint16_t *out) {
  const int Wp = W + 2;
  for (int ty = 0; ty < H / 2; ty++)
    for (int tx = 0; tx < W / 2; tx++) {
      const uint16_t *d = x + ((size_t)(2 * ty) * Wp + 2 * tx) * 24;
      for (int co = 0; co < 24; co++) {
        uint16_t M[16];
        for (int p = 0; p < 16; p++) M[p] = 0;
        for (int ci = 0; ci < 24; ci++) {
          uint16_t dd[4][4], t[4][4], V[16];
          for (int r = 0; r < 4; r++)
            for (int j = 0; j < 4; j++) dd[r][j] = d[((size_t)r * Wp + j) * 24 + ci];
          for (int j = 0; j < 4; j++) {
            t[0][j] = HSUB(dd[0][j], dd[2][j]); t[1][j] = HADD(dd[1][j], dd[2][j]);
            t[2][j] = HSUB(dd[2][j], dd[1][j]); t[3][j] = HSUB(dd[1][j], dd[3][j]);
          }
          for (int i = 0; i < 4; i++) {
            V[i * 4 + 0] = HSUB(t[i][0], t[i][2]); V[i * 4 + 1] = HADD(t[i][1], t[i][2]);
            V[i * 4 + 2] = HSUB(t[i][2], t[i][1]); V[i * 4 + 3] = HSUB(t[i][1], t[i][3]);
          }
          /* gemm4: per position, an fp16 FMA chain over ci in order, from zero (FMLA by element) */
          for (int p = 0; p < 16; p++) M[p] = orc_h_fma(U[((size_t)p * 24 + ci) * 24 + co], V[p], M[p]);
        }
        uint16_t s[2][4], y[4];
        for (int j = 0; j < 4; j++) {
          s[0][j] = HADD(HADD(M[j], M[4 + j]), M[8 + j]);
          s[1][j] = HSUB(HSUB(M[4 + j], M[8 + j]), M[12 + j]);
        }
        for (int i = 0; i < 2; i++) {
          y[2 * i] = HADD(HADD(HADD(s[i][0], s[i][1]), s[i][2]), b16[co]);
          y[2 * i + 1] = HADD(HSUB(HSUB(s[i][1], s[i][2]), s[i][3]), b16[co]);
        }
        for (int q = 0; q < 4; q++) {
          const int i = q / 2, j = q % 2;
          const size_t off = ((size_t)(2 * ty + 1 + i) * Wp + 2 * tx + 1 + j) * 24 + co;
          out[off] = HADD(orc_silu_poly_h(y[q]), x[off]);
        }
      }
    }
}
