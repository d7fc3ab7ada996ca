/* CPU oracle (test infrastructure only; never linked into the product): AArch64 scalar semantics, the int8
 * no-dotprod GEMM of libbnneon (PW_S8) and this project's Q31 requantised GEMM specification. See oracle.h. */
#include <math.h>
#include <string.h>

#include "oracle.h"

static inline uint32_t fbits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float bitsf(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* ---------------------------------------------------------------- AArch64 scalar semantics */

/* RecipEstimate of the Arm ARM (single-precision table lookup replaced by the integer formula it is defined by):
 * a in [256, 512) is 1.fraction<51:44> scaled by 2^8; returns r in [256, 512) representing r / 256. */
int orc_recip_estimate(int a) {
  a = a * 2 + 1;
  int b = (1 << 19) / a;
  return (b + 1) / 2;
}

/* FPRecipEstimate (Arm ARM, shared/functions/float/fprecipestimate) for N = 32 with FPCR.FZ = 0, RMode = RN. */
float orc_frecpe(float x) {
  uint32_t u = fbits(x), sign = u & 0x80000000u, exp = (u >> 23) & 0xffu, frac = u & 0x7fffffu;
  if (exp == 0xffu && frac) return bitsf(u | 0x400000u);           /* NaN: quieted operand */
  if (exp == 0xffu) return bitsf(sign);                            /* +-inf -> +-0 */
  if (exp == 0 && frac == 0) return bitsf(sign | 0x7f800000u);     /* +-0 -> +-inf (divide by zero) */
  if (exp == 0 && frac < 0x200000u) return bitsf(sign | 0x7f800000u); /* |x| < 2^-128: overflow, RN -> inf */
  uint64_t fraction = (uint64_t)frac << 29;                         /* 52-bit fraction field */
  int e = (int)exp;
  if (e == 0) {                                                     /* denormal operand */
    if (!((fraction >> 51) & 1)) { e = -1; fraction = (fraction & ((1ull << 50) - 1)) << 2; }
    else fraction = (fraction & ((1ull << 51) - 1)) << 1;
  }
  int scaled = 256 | (int)((fraction >> 44) & 0xffu);
  int result_exp = 253 - e;
  int est = orc_recip_estimate(scaled);
  fraction = (uint64_t)(est & 0xff) << 44;
  if (result_exp == 0) fraction = (1ull << 51) | (fraction >> 1);
  else if (result_exp == -1) { fraction = (1ull << 50) | (fraction >> 2); result_exp = 0; }
  return bitsf(sign | ((uint32_t)(result_exp & 0xff) << 23) | (uint32_t)((fraction >> 29) & 0x7fffffu));
}

/* FPRecipStepFused: 2 - a*b with one rounding; (inf, 0) and (0, inf) give +2 */
float orc_frecps(float a, float b) {
  if (isnan(a) || isnan(b)) return isnan(a) ? bitsf(fbits(a) | 0x400000u) : bitsf(fbits(b) | 0x400000u);
  if ((isinf(a) && b == 0.f) || (a == 0.f && isinf(b))) return 2.f;
  if (isinf(a) || isinf(b)) return ((signbit(a) != 0) ^ (signbit(b) != 0)) ? INFINITY : -INFINITY;
  return fmaf(-a, b, 2.f);
}

float orc_fmax(float a, float b) {
  if (isnan(a)) return bitsf(fbits(a) | 0x400000u);
  if (isnan(b)) return bitsf(fbits(b) | 0x400000u);
  if (a == 0.f && b == 0.f) return (signbit(a) && signbit(b)) ? -0.f : 0.f;
  return a > b ? a : b;
}
float orc_fmin(float a, float b) {
  if (isnan(a)) return bitsf(fbits(a) | 0x400000u);
  if (isnan(b)) return bitsf(fbits(b) | 0x400000u);
  if (a == 0.f && b == 0.f) return (signbit(a) || signbit(b)) ? -0.f : 0.f;
  return a < b ? a : b;
}

static int32_t sat_s32(float r) { /* r integral (or NaN / inf) */
  if (r != r) return 0;
  if (r >= 2147483648.f) return INT32_MAX;
  if (r < -2147483648.f) return INT32_MIN;
  return (int32_t)r;
}
int32_t orc_cvtn_s32(float x) { return sat_s32(rintf(x)); }
int32_t orc_cvta_s32(float x) { return sat_s32(roundf(x)); }
int32_t orc_cvtz_s32(float x) { return sat_s32(truncf(x)); }
int32_t orc_lrintf_s32(float x) {
  float r = rintf(x);
  int64_t v;
  if (r != r) v = 0;
  else if (r >= 9223372036854775808.f) v = INT64_MAX;
  else if (r < -9223372036854775808.f) v = INT64_MIN;
  else v = (int64_t)r;
  return (int32_t)(uint32_t)(uint64_t)v;
}

/* src/gemm_f32.h:102-118 (silu_f32x4); silu4_f32x4 (:122-145) is the same chain per lane */
float orc_silu_f32(float x) {
  const float magic = 12582912.0f;
  float t = x * -1.44269504f;
  t = orc_fmin(orc_fmax(t, -60.f), 60.f);
  float tm = t + magic;
  float f = t - (tm - magic);
  uint32_t ni = fbits(tm) << 23;
  float p = fmaf(1.3333558e-3f, f, 9.6181291e-3f);
  p = fmaf(p, f, 5.5504109e-2f);
  p = fmaf(p, f, 2.4022651e-1f);
  p = fmaf(p, f, 6.9314718e-1f);
  p = fmaf(p, f, 1.0f);
  float d = 1.f + bitsf(fbits(p) + ni);
  float r = orc_frecpe(d);
  r = r * orc_frecps(d, r);
  return x * r;
}

/* ---------------------------------------------------------------- PW_S8 */

/* src/gemm_s8n.c:15-51. The 4-lane min / max (FMIN / FMAX, NaN-propagating) over k < K & ~3, then the scalar tail
 * with fminf / fmaxf (FMINNM / FMAXNM: a NaN operand is ignored); the 8-wide quantization loop converts with FCVTNS
 * (int32-saturating), the scalar tail with (int32_t)lrintf (64-bit saturating, truncated). */
void orc_s8n_quant_rows(const float *x, int ld, int r0, int r1, int K, int Kp, int8_t *q, float *sa, int32_t *za) {
  for (int m = r0; m < r1; m++) {
    const float *r = x + (size_t)m * ld;
    float mn[4] = {INFINITY, INFINITY, INFINITY, INFINITY}, mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    int k = 0;
    for (; k + 4 <= K; k += 4)
      for (int j = 0; j < 4; j++) { mn[j] = orc_fmin(mn[j], r[k + j]); mx[j] = orc_fmax(mx[j], r[k + j]); }
    float lo = orc_fmin(orc_fmin(mn[0], mn[1]), orc_fmin(mn[2], mn[3]));
    float hi = orc_fmax(orc_fmax(mx[0], mx[1]), orc_fmax(mx[2], mx[3]));
    for (; k < K; k++) { lo = fminf(lo, r[k]); hi = fmaxf(hi, r[k]); }
    int8_t *o = q + (size_t)m * Kp;
    float inv;
    int32_t z;
    float range = hi - lo;
    if (!(range > 1e-30f * fmaxf(fabsf(hi), fabsf(lo))) || !(range > 0.f)) {
      float a = fmaxf(fabsf(hi), 1e-30f);
      inv = 127.f / a; z = 0; sa[m] = a / 127.f;
    } else {
      inv = 254.f / range;
      z = (int32_t)((uint32_t)-127 - (uint32_t)orc_lrintf_s32(lo * inv));
      sa[m] = range / 254.f;
    }
    za[m] = z;
    k = 0;
    for (; k + 8 <= K; k += 8)
      for (int j = 0; j < 8; j++) {
        int32_t v = (int32_t)((uint32_t)orc_cvtn_s32(r[k + j] * inv) + (uint32_t)z);
        o[k + j] = (int8_t)(v < -127 ? -127 : v > 127 ? 127 : v);
      }
    for (; k < K; k++) {
      int32_t v = (int32_t)((uint32_t)orc_lrintf_s32(r[k] * inv) + (uint32_t)z);
      o[k] = (int8_t)(v < -127 ? -127 : v > 127 ? 127 : v);
    }
    for (; k < Kp; k++) o[k] = (int8_t)(uint8_t)((uint32_t)z & 0xffu);
  }
}

/* src/gemm_s8n.c:55-63: each row gated (one fp32 multiply per element), then quantized as above */
void orc_s8n_quant_rows_gate(const float *x, int ld, int r0, int r1, int K, int Kp, const float *gate, int8_t *q,
                             float *sa, int32_t *za) {
  float t[4096];
  for (int m = r0; m < r1; m++) {
    const float *r = x + (size_t)m * ld;
    for (int k = 0; k < K; k++) t[k] = r[k] * gate[k];
    /* quantize the one gated row as row m (the reference passes ld 0 and row m of t) */
    orc_s8n_quant_rows(t, 0, m, m + 1, K, Kp, q, sa, za);
  }
}

static size_t orow(const orc_epi32 *e, int m) {
  if (!e->opad) return (size_t)m;
  return (size_t)((m / e->ow) + e->opad) * (e->ow + 2 * e->opad) + (m % e->ow) + e->opad;
}
static size_t rrow(const orc_epi32 *e, int m) {
  if (!e->rpad) return (size_t)m;
  return (size_t)((m / e->rw) + e->rpad) * (e->rw + 2 * e->rpad) + (m % e->rw) + e->rpad;
}

/* src/gemm_s8n.c:82-135 (acc4x4, deq4, activation, store_rows): exact int32 sums (two's complement), the zero-point
 * correction in wrapping int32, an RNE int->float conversion, y = f * (sw * sa) + b as three roundings, SiLU or
 * ReLU (FMAX with +0), the residual added after the activation. */
void orc_s8n_gemm(const int8_t *q, int Kp, const float *sa, const int32_t *za, int M, int Np, const int8_t *w,
                  const float *sw, const int32_t *colsum, const float *b, const orc_epi32 *e) {
  const int kb = Kp / 16;
  for (int m = 0; m < M; m++) {
    const int8_t *a = q + (size_t)m * Kp;
    for (int n = 0; n < Np; n++) {
      const int8_t *wp = w + (size_t)(n / 4) * kb * 64 + (n % 4) * 16;
      uint32_t acc = 0;
      for (int k = 0; k < Kp; k++) acc += (uint32_t)((int32_t)a[k] * (int32_t)wp[(size_t)(k / 16) * 64 + k % 16]);
      int32_t c = (int32_t)(acc - (uint32_t)colsum[n] * (uint32_t)za[m]);
      float f = (float)c;
      float s = sw[n] * sa[m];
      float y = f * s;
      y = y + b[n];
      if (e->act == 1) y = orc_silu_f32(y);
      else if (e->act == 2) y = orc_fmax(y, 0.f);
      if (e->res) y = y + e->res[rrow(e, m) * e->ldr + n];
      e->out[orow(e, m) * e->ldo + n] = y;
    }
  }
}

void orc_zero_halo(void *xp, int H, int W, int C, int h, size_t esz) {
  char *x = xp;
  size_t rowl = (size_t)(W + 2 * h) * C * esz, side = (size_t)C * h * esz;
  memset(x, 0, rowl * h);
  memset(x + (size_t)(H + h) * rowl, 0, rowl * h);
  for (int y = h; y < H + h; y++) {
    memset(x + (size_t)y * rowl, 0, side);
    memset(x + (size_t)y * rowl + (size_t)(W + h) * C * esz, 0, side);
  }
}

void orc_pw_s8(const float *in, int lda, int M, int K, int Kp, int N, int Np, const float *gate, int8_t *q, float *sa,
               int32_t *za, const int8_t *w, const float *sw, const int32_t *colsum, const float *b, const orc_epi32 *e) {
  (void)N;
  if (e->opad) orc_zero_halo(e->out, M / e->ow, e->ow, e->ldo, e->opad, 4);
  if (gate) orc_s8n_quant_rows_gate(in, lda, 0, M, K, Kp, gate, q, sa, za);
  else orc_s8n_quant_rows(in, lda, 0, M, K, Kp, q, sa, za);
  orc_s8n_gemm(q, Kp, sa, za, M, Np, w, sw, colsum, b, e);
}

/* ---------------------------------------------------------------- Q31 requant (own specification, oracle.h) */
int32_t orc_srdhm(int32_t a, int32_t b) {
  if (a == INT32_MIN && b == INT32_MIN) return INT32_MAX;
  int64_t ab = (int64_t)a * (int64_t)b;
  int64_t nudge = ab >= 0 ? (1LL << 30) : (1 - (1LL << 30));
  return (int32_t)((ab + nudge) / (1LL << 31));
}
int32_t orc_rdbypot(int32_t x, int e) {
  int32_t mask = (int32_t)((1u << e) - 1u);
  int32_t rem = x & mask;
  int32_t thr = (mask >> 1) + (x < 0 ? 1 : 0);
  return (x >> e) + (rem > thr ? 1 : 0);
}
int8_t orc_requant(int32_t acc, int32_t mult, int shift, int zy, int lo, int hi) {
  int32_t y = orc_rdbypot(orc_srdhm(acc, mult), shift);
  int64_t v = (int64_t)y + zy;
  return (int8_t)(v < lo ? lo : v > hi ? hi : v);
}
void orc_gemm_s8_requant(const int8_t *w, const int8_t *x, const int32_t *bias, const int32_t *mult, const int32_t *shift,
                         int N, int K, int M, int zx, int zy, int lo, int hi, int8_t *out) {
  for (int n = 0; n < N; n++)
    for (int m = 0; m < M; m++) {
      uint32_t acc = (uint32_t)bias[n];
      for (int k = 0; k < K; k++) acc += (uint32_t)((int32_t)w[(size_t)n * K + k] * ((int32_t)x[(size_t)k * M + m] - zx));
      out[(size_t)n * M + m] = orc_requant((int32_t)acc, mult[n], shift[n], zy, lo, hi);
    }
}

/* y[i] = f(x[i]): 0 FRECPE, 1 the epilogue SiLU, 2 ReLU (FMAX with +0); the batch form of the checks above */
void orc_eval_f32(int f, const float *x, float *y, long long n) {
  for (long long i = 0; i < n; i++) y[i] = f == 0 ? orc_frecpe(x[i]) : f == 1 ? orc_silu_f32(x[i]) : orc_fmax(x[i], 0.f);
}
