/* CPU oracle of the dotprod family's int8 arithmetic (QPW, QCONV3, HEADS_S8, SE_GATE16, GEM_A): test infrastructure
 * only (see oracle.h). Asymmetric per-row (or per-tensor) activation quantisation to [-128, 127] with a float zero
 * point, symmetric per-channel weights in [-127, 127], exact int32 sums and the fp32 FMA epilogue
 * v = (b + (f sw) sa) + swsum (sa zp), both sums fused. Weights are kept here as plain rows q [N][Kp] (Kp = K rounded
 * up to 16, zero past K): the oracle's own layout; the reference's c4 panels hold the same values. */
#include <math.h>
#include <float.h>
#include <string.h>

#include "oracle.h"

static uint32_t fb(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float bf(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* qw_pack (src/gemm_s8.c:10-35): per output channel s = max|w| / 127 (1 when all zero), q = clamp(rint(w / s), +-127),
 * swsum = s * (float)sum q */
void orc_qd_wpack(const float *w, const float *bias, int N, int K, int8_t *q, float *scale, float *swsum, float *b) {
  const int Kp = (K + 15) & ~15;
  memset(q, 0, (size_t)N * Kp);
  for (int n = 0; n < N; n++) {
    const float *r = w + (size_t)n * K;
    float mx = 0;
    for (int k = 0; k < K; k++) mx = fmaxf(mx, fabsf(r[k]));
    const float s = mx > 0 ? mx / 127.f : 1.f;
    scale[n] = s;
    b[n] = bias ? bias[n] : 0.f;
    int32_t sum = 0;
    for (int k = 0; k < K; k++) {
      int v = (int)nearbyintf(r[k] / s);
      v = v > 127 ? 127 : (v < -127 ? -127 : v);
      sum += v;
      q[(size_t)n * Kp + k] = (int8_t)v;
    }
    swsum[n] = s * (float)sum;
  }
}

/* params (src/gemm_s8.c:295-304): the range always holds 0; zp = rint(mn / s) + 128 */
void orc_qd_params(float mn, float mx, float *scale, float *zp, float *inv) {
  mn = fminf(mn, 0.f);
  mx = fmaxf(mx, 0.f);
  const float s = (mx - mn) > 0 ? (mx - mn) / 255.f : 1.f;
  const float iv = 1.f / s;
  *scale = s;
  *zp = nearbyintf(mn * iv) + 128.f;
  *inv = iv;
}

/* q8_f32x8 lane (src/gemm_s8.c:284-293): the bits of fma(x, inv, 1.5 * 2^23) minus 0x4B400000 + zp, clamped */
static int8_t q8_magic(float x, float inv, int32_t zofs) {
  int32_t q = (int32_t)(fb(fmaf(x, inv, 12582912.0f)) - (uint32_t)zofs);
  return (int8_t)(q > 127 ? 127 : (q < -128 ? -128 : q));
}
static int8_t q8_tail(float v, float zp) {
  const float q = nearbyintf(v) - zp;
  return (int8_t)(q > 127 ? 127 : (q < -128 ? -128 : q));
}

/* quant_rows_f32 (src/gemm_s8.c:349-371). rq [M][2] = {scale, zp}. The 4-lane FMIN / FMAX from 0 over k < C & ~3 (the
 * lane split and FMINV order cannot change a NaN-propagating min), FMINNM / FMAXNM over the tail; magic-number
 * quantisation over k < C & ~7, rint over the tail; zeros to Cp. */
void orc_qd_quant_rows_f32(const float *x, int ldx, int M, int C, int8_t *a, int lda, int Cp, float *rq) {
  for (int m = 0; m < M; m++) {
    const float *r = x + (size_t)m * ldx;
    int8_t *o = a + (size_t)m * lda;
    float mn = 0.f, mx = 0.f;
    int c = 0;
    for (; c < (C & ~3); c++) { mn = orc_fmin(mn, r[c]); mx = orc_fmax(mx, r[c]); }
    for (; c < C; c++) { mn = fminf(mn, r[c]); mx = fmaxf(mx, r[c]); }
    float s, zp, inv;
    orc_qd_params(mn, mx, &s, &zp, &inv);
    rq[2 * m] = s;
    rq[2 * m + 1] = zp;
    const int32_t zofs = 0x4B400000 + (int32_t)zp;
    c = 0;
    for (; c < (C & ~7); c++) o[c] = q8_magic(r[c], inv, zofs);
    for (; c < C; c++) o[c] = q8_tail(r[c] * inv, zp);
    for (; c < Cp; c++) o[c] = 0;
  }
}

/* quant_rows_f16 (src/gemm_s8.c:306-347): all-fp16 arithmetic over k < C & ~7 for the range (the gated product
 * rounded to fp16) and over k < C & ~15 for the quantisation (fma(h, (fp16)inv, 1536) in fp16, its bits minus
 * 0x6600 + zp in wrapping int16, clamped); the tails in fp32 with the unrounded inv. */
void orc_qd_quant_rows_f16(const uint16_t *x, int ldx, int M, int C, const uint16_t *gate, int8_t *a, int lda, int Cp,
                           float *rq) {
  for (int m = 0; m < M; m++) {
    const uint16_t *r = x + (size_t)m * ldx;
    int8_t *o = a + (size_t)m * lda;
    uint16_t mnh = 0, mxh = 0;
    int c = 0;
    for (; c < (C & ~7); c++) {
      const uint16_t h = gate ? orc_h_mul(r[c], gate[c]) : r[c];
      mnh = orc_h_min(mnh, h);
      mxh = orc_h_max(mxh, h);
    }
    float fmn = orc_h2f(mnh), fmx = orc_h2f(mxh);
    for (; c < C; c++) {
      const float v = orc_h2f(r[c]) * (gate ? orc_h2f(gate[c]) : 1.f);
      fmn = fminf(fmn, v);
      fmx = fmaxf(fmx, v);
    }
    float s, zp, inv;
    orc_qd_params(fmn, fmx, &s, &zp, &inv);
    rq[2 * m] = s;
    rq[2 * m + 1] = zp;
    const uint16_t hinv = orc_f2h(inv);
    const int16_t zo = (int16_t)(0x6600 + (int)zp);
    c = 0;
    for (; c < (C & ~15); c++) {
      const uint16_t h = gate ? orc_h_mul(r[c], gate[c]) : r[c];
      int16_t q = (int16_t)(uint16_t)(orc_h_fma(h, hinv, 0x6600) - (uint16_t)zo);
      q = q < -128 ? -128 : (q > 127 ? 127 : q);
      o[c] = (int8_t)q;
    }
    for (; c < C; c++) o[c] = q8_tail(orc_h2f(r[c]) * (gate ? orc_h2f(gate[c]) : 1.f) * inv, zp);
    for (; c < Cp; c++) o[c] = 0;
  }
}

/* exp2_p5_f32 lane (src/act.h:9-21): magic-number split t = n + f, degree-5 polynomial, n added to the exponent bits */
float orc_exp2_p5(float t) {
  const float magic = 12582912.0f;
  const float tm = t + magic, n = tm - magic, f = t - n;
  const uint32_t ni = fb(tm) << 23;
  float p = fmaf(1.3333558e-3f, f, 9.6181291e-3f);
  p = fmaf(p, f, 5.5504109e-2f);
  p = fmaf(p, f, 2.4022651e-1f);
  p = fmaf(p, f, 6.9314718e-1f);
  p = fmaf(p, f, 1.0f);
  return bf(fb(p) + ni);
}

/* silu_f32_a lane (src/act.h:41-49): t clamped to [-126, 126], FRECPE and two Newton steps */
float orc_silu_f32_a(float x) {
  float t = x * -1.44269504f;
  t = orc_fmin(orc_fmax(t, -126.f), 126.f);
  const float d = orc_exp2_p5(t) + 1.0f;
  float r = orc_frecpe(d);
  r = r * orc_frecps(d, r);
  r = r * orc_frecps(d, r);
  return x * r;
}

/* log2_f32 lane (src/act.h:23-38): exponent + atanh series of the mantissa shifted to [sqrt(.5), sqrt(2)) */
float orc_log2_dot(float x) {
  const int32_t xi = (int32_t)fb(x);
  const int32_t t = (int32_t)((uint32_t)xi - 0x3F3504F3u);
  const int32_t e = t >> 23;
  const float mnt = bf((uint32_t)xi - ((uint32_t)e << 23));
  const float z = mnt - 1.0f;
  const float u = z / (mnt + 1.0f);
  const float u2 = u * u;
  float pp = fmaf(u2, 1.f / 9, 1.f / 7);
  pp = fmaf(pp, u2, 1.f / 5);
  pp = fmaf(pp, u2, 1.f / 3);
  pp = fmaf(pp, u2, 1.f);
  const float ln = (u * 2.f) * pp;
  return fmaf(ln, 1.44269504f, (float)e);
}

static size_t opix(const orc_qd_epi *e, int m) {
  if (!e->opad) return (size_t)m;
  const int y = m / e->ow, x = m - y * e->ow;
  return (size_t)(y + e->opad) * (e->ow + 2 * e->opad) + x + e->opad;
}

/* gemm_s8 (src/gemm_s8.c:54-87 tile_row, :143-150 affine4, :153-278 gemm_core): f = (float)acc (exact or RNE),
 * v = fma(swsum, sa zp, fma(f sw, sa, b)); fp16 out: v rounded to fp16, then the table SiLU; fp32 out: silu_f32_a
 * or FMAX with 0, then + the residual (rows m, stride ldo). rq: per row [M][2], or one pair when per_tensor. */
void orc_qd_gemm(const int8_t *a, int lda, const float *rq, int per_tensor, int M, int N, int Kp, const int8_t *q,
                 const float *scale, const float *swsum, const float *b, const orc_qd_epi *e) {
  for (int m = 0; m < M; m++) {
    const float sa = per_tensor ? rq[0] : rq[2 * m], zp = per_tensor ? rq[1] : rq[2 * m + 1];
    const float zs = sa * zp;
    const int8_t *ar = a + (size_t)m * lda;
    for (int n = 0; n < N; n++) {
      const int8_t *wr = q + (size_t)n * Kp;
      int64_t acc = 0;
      for (int k = 0; k < Kp; k++) acc += (int32_t)ar[k] * (int32_t)wr[k];
      const float f = (float)(int32_t)acc;
      const float v0 = f * scale[n];
      const float v = fmaf(swsum[n], zs, fmaf(v0, sa, b[n]));
      const size_t po = opix(e, m) * e->ldo + n;
      if (e->out16) {
        uint16_t h = orc_f2h(v);
        if (e->act == 1) h = orc_silu_lut_h(h);
        e->out16[po] = h;
      } else {
        float y = v;
        if (e->act == 1) y = orc_silu_f32_a(y);
        else if (e->act == 2) y = orc_fmax(y, 0.f);
        if (e->res32) y = y + e->res32[(size_t)m * e->ldo + n];
        e->out32[po] = y;
      }
    }
  }
}

/* QPW (src/rt_ops_dot.c:326-339 with rows_range :270-281): quantise every row (fp32, or fp16 gated), then the GEMM.
 * a8 [M][Kp] and rq [M][2] are written as the op's buffers. */
void orc_qpw(const void *x, int in_f16, int ldx, int M, int K, const uint16_t *gate, int8_t *a8, float *rq, int N,
             const int8_t *q, const float *scale, const float *swsum, const float *b, const orc_qd_epi *e) {
  const int Kp = (K + 15) & ~15;
  if (in_f16) orc_qd_quant_rows_f16((const uint16_t *)x, ldx, M, K, gate, a8, Kp, Kp, rq);
  else orc_qd_quant_rows_f32((const float *)x, ldx, M, K, a8, Kp, Kp, rq);
  orc_qd_gemm(a8, Kp, rq, 0, M, N, Kp, q, scale, swsum, b, e);
}

/* quant_tensor_pad_f32 (src/gemm_s8.c:373-396): one (scale, zp) for the whole H x W x C tensor, a one-pixel halo of
 * the zero point's code (-zp) around the magic-number codes */
void orc_qd_quant_tensor_pad(const float *x, int H, int W, int C, int8_t *out, float *rq) {
  const size_t n = (size_t)H * W * C;
  float mn = 0.f, mx = 0.f;
  for (size_t i = 0; i < n; i++) { mn = orc_fmin(mn, x[i]); mx = orc_fmax(mx, x[i]); }
  float s, zp, inv;
  orc_qd_params(mn, mx, &s, &zp, &inv);
  rq[0] = s;
  rq[1] = zp;
  const int8_t halo = (int8_t)(-(int)zp);
  const int32_t zofs = 0x4B400000 + (int32_t)zp;
  const int Wp = W + 2;
  for (int y = 0; y < H + 2; y++)
    for (int xx = 0; xx < Wp; xx++)
      for (int c = 0; c < C; c++) {
        int8_t v = halo;
        if (y >= 1 && y <= H && xx >= 1 && xx <= W) v = q8_magic(x[((size_t)(y - 1) * W + xx - 1) * C + c], inv, zofs);
        out[((size_t)y * Wp + xx) * C + c] = v;
      }
}

/* QCONV3 (src/rt_ops_dot.c:177-216 with im2col_s8, src/gemm_s8.c:398-418): 3x3 stride s TF-same conv (low pads pt,
 * pl) over the per-tensor quantised padded copy, the GEMM with SiLU into fp16 rows [Ho*Wo][K]. xp: scratch of
 * (H+2)(W+2)C bytes; col: scratch of Ho*Wo*Kp bytes. */
void orc_qconv3(const float *x, int H, int W, int C, int K, int s, int pt, int pl, int Ho, int Wo, const int8_t *q,
                const float *scale, const float *swsum, const float *b, int8_t *xp, int8_t *col, uint16_t *out) {
  float rq[2];
  orc_qd_quant_tensor_pad(x, H, W, C, xp, rq);
  const int Kp = (9 * C + 15) & ~15, Wp = W + 2;
  for (int oy = 0; oy < Ho; oy++)
    for (int ox = 0; ox < Wo; ox++) {
      int8_t *d = col + ((size_t)oy * Wo + ox) * Kp;
      for (int ky = 0; ky < 3; ky++) {
        const int8_t *row = xp + ((size_t)(oy * s + ky - pt + 1) * Wp + (ox * s - pl + 1)) * C;
        memcpy(d + ky * 3 * C, row, (size_t)3 * C);
      }
      memset(d + 9 * C, 0, (size_t)(Kp - 9 * C));
    }
  orc_qd_epi e = {.act = 1, .out16 = out, .ldo = K};
  orc_qd_gemm(col, Kp, rq, 1, Ho * Wo, K, Kp, q, scale, swsum, b, &e);
}

/* SE_GATE16 (src/rt_ops_dot.c:381-420): chsum scaled to means in place (x * (1/P)); fc1 from fp16-held weights:
 * two 4-lane fp32 FMA accumulators over 8-channel steps (lanes 0-3, 4-7), lane pairs added, then the 4 lanes pairwise
 * ((l0 + l1) + (l2 + l3)), + b1, SiLU v / (1 + expf(-v)) with the C library's expf; fc2 from b2, one FMA per r with
 * fp16-held weights; sigmoid by exp2_p5 (t clamped to +-126), FRECPE and two Newton steps; rounded to fp16.
 * w1 [rd][C], w2 [C][rd] as fp32 (rounded to fp16 here, as the op's init does). */
void orc_se_gate16(float *chsum, int C, int rd, int P, const float *w1, const float *b1, const float *w2,
                   const float *b2, uint16_t *gate) {
  const float inv = 1.f / P;
  for (int ch = 0; ch < C; ch++) chsum[ch] *= inv;
  float tmp[4096];
  orc_se_fc1(chsum, C, rd, w1, 1, b1, tmp);
  for (int ch = 0; ch < C; ch++) {
    float g = b2[ch];
    for (int r = 0; r < rd; r++) g = fmaf(orc_h2f(orc_f2h(w2[(size_t)ch * rd + r])), tmp[r], g);
    const float t = orc_fmin(orc_fmax(g * -1.44269504f, -126.f), 126.f);
    const float d = orc_exp2_p5(t) + 1.f;
    float r0 = orc_frecpe(d);
    r0 = r0 * orc_frecps(d, r0);
    r0 = r0 * orc_frecps(d, r0);
    gate[ch] = orc_f2h(r0);
  }
}

/* GEM_A (src/rt_ops_dot.c:439-465): e[c] = powf(mean over rows of exp2_p5(max(p log2(max(F, eps)), -126)), 1/p), the
 * sums in row order from 0, powf the C library's */
void orc_gem_a(const float *F, int M, int C, float eps, float p, float *e) {
  for (int ch = 0; ch < C; ch++) {
    float acc = 0.f;
    for (int i = 0; i < M; i++) {
      const float v = orc_fmax(F[(size_t)i * C + ch], eps);
      acc = acc + orc_exp2_p5(orc_fmax(p * orc_log2_dot(v), -126.f));
    }
    e[ch] = powf(acc / M, 1.0f / p);
  }
}

/* HEADS_S8's pooling of one head (src/rt_ops_dot.c:531-550): i = 0, per time step t < H the mean over W of F
 * [H*W][C]; i = 1, per t < W the mean over H; each a sum from 0 in order of the other axis, divided by its length;
 * then per t max-pool 3 (fmaxf from -FLT_MAX) + average-pool 3 (sum from 0 of v * 0.33333334f, multiply then add,
 * in order of t - 1, t, t + 1, edges skipped): s [L][C] the means, pooled [L][C] */
void orc_heads_pool(const float *F, int H, int W, int C, int i, float *s, float *pooled) {
  const int Lt = i == 0 ? H : W;
  for (int t = 0; t < Lt; t++)
    for (int ch = 0; ch < C; ch++) {
      float a2 = 0;
      if (i == 0) {
        for (int u = 0; u < W; u++) a2 += F[(size_t)(t * W + u) * C + ch];
        s[t * C + ch] = a2 / W;
      } else {
        for (int u = 0; u < H; u++) a2 += F[(size_t)(u * W + t) * C + ch];
        s[t * C + ch] = a2 / H;
      }
    }
  for (int t = 0; t < Lt; t++)
    for (int ch = 0; ch < C; ch++) {
      float mx = -FLT_MAX, sum = 0;
      for (int d = -1; d <= 1; d++) {
        const int u = t + d;
        if (u < 0 || u >= Lt) continue;
        const float v = s[u * C + ch];
        mx = fmaxf(mx, v);
        sum += v * 0.33333334f;
      }
      pooled[t * C + ch] = mx + sum;
    }
}

/* HEADS_S8's attention pooling of one head (src/rt_ops_dot.c:559-570): per class k < nc, att [L][ncp] clipped to
 * [-10, 10] in place, mx = fmaxf over t from -FLT_MAX; then in order of t from 0: ev = expf(att - mx) (the C
 * library's), z += ev, acc += ev * cla (multiply, then add); logits[k] += acc / z */
void orc_heads_softmax(float *att, const float *cla, int L, int nc, int ncp, float *logits) {
  for (int k = 0; k < nc; k++) {
    float mx = -FLT_MAX;
    for (int t = 0; t < L; t++) {
      float a2 = att[(size_t)t * ncp + k];
      a2 = a2 < -10.f ? -10.f : (a2 > 10.f ? 10.f : a2);
      att[(size_t)t * ncp + k] = a2;
      mx = fmaxf(mx, a2);
    }
    float z = 0, acc = 0;
    for (int t = 0; t < L; t++) {
      const float ev = expf(att[(size_t)t * ncp + k] - mx);
      z += ev;
      acc += ev * cla[(size_t)t * ncp + k];
    }
    logits[k] += acc / z;
  }
}

/* HEADS_S8 (src/rt_ops_dot.c:520-572). logits [ncp] = lin(e) (int8 GEMM, 1 row), then for the head over H (i = 0:
 * per time step t < H the mean over W) and over W (i = 1: per t < W the mean over H): max-pool 3 + average-pool 3
 * (weights 0.33333334, zero-padded) of the means, fc + ReLU, att and cla (int8 GEMMs with per-row quantised inputs),
 * att clipped to [-10, 10], soft-max over t with the C library's expf, logits[k] += sum(ev cla) / sum(ev), k < nc.
 * The weights: 7 matrices of ncp / hid output rows as orc_qd_wpack wrote them, in the order lin, fc0, att0, cla0, fc1,
 * att1, cla1 (wq[i], sc[i], ss[i], bb[i]); work: scratch of 4 (L + 4) max(C, hid, ncp) floats + (L + 4) max(C, hid)
 * bytes, L = max(H, W). */
void orc_heads_s8(const float *F, const float *emb, int H, int W, int C, int hid, int nc, const int8_t *const *wq,
                  const float *const *sc, const float *const *ss, const float *const *bb, float *logits, float *work) {
  const int ncp = (nc + 15) & ~15, L = H > W ? H : W, Kc = (C + 15) & ~15, Kh = (hid + 15) & ~15;
  const int wmax = C > hid ? (C > ncp ? C : ncp) : (hid > ncp ? hid : ncp);
  float *s = work, *pooled = s + (size_t)(L + 4) * wmax, *h = pooled + (size_t)(L + 4) * wmax;
  float *att = h + (size_t)(L + 4) * wmax, *cla = att + (size_t)(L + 4) * wmax;
  int8_t *a8 = (int8_t *)(cla + (size_t)(L + 4) * wmax);
  float rq[2 * 4096];
  orc_qd_quant_rows_f32(emb, C, 1, C, a8, Kc, Kc, rq);
  orc_qd_epi el = {.act = 0, .out32 = logits, .ldo = ncp};
  orc_qd_gemm(a8, Kc, rq, 0, 1, ncp, Kc, wq[0], sc[0], ss[0], bb[0], &el);
  for (int i = 0; i < 2; i++) {
    const int Lt = i == 0 ? H : W, j = 1 + 3 * i;
    orc_heads_pool(F, H, W, C, i, s, pooled);
    orc_qd_quant_rows_f32(pooled, C, Lt, C, a8, Kc, Kc, rq);
    orc_qd_epi ef = {.act = 2, .out32 = h, .ldo = hid};
    orc_qd_gemm(a8, Kc, rq, 0, Lt, hid, Kc, wq[j], sc[j], ss[j], bb[j], &ef);
    orc_qd_quant_rows_f32(h, hid, Lt, hid, a8, Kh, Kh, rq);
    orc_qd_epi ea = {.act = 0, .out32 = att, .ldo = ncp};
    orc_qd_gemm(a8, Kh, rq, 0, Lt, ncp, Kh, wq[j + 1], sc[j + 1], ss[j + 1], bb[j + 1], &ea);
    orc_qd_epi ec = {.act = 0, .out32 = cla, .ldo = ncp};
    orc_qd_gemm(a8, Kh, rq, 0, Lt, ncp, Kh, wq[j + 2], sc[j + 2], ss[j + 2], bb[j + 2], &ec);
    orc_heads_softmax(att, cla, Lt, nc, ncp, logits);
  }
}

/* the C library's powf elementwise (the reference of GEM_A's final power, src/rt_ops_dot.c:452) */
void orc_powf_vec(const float *x, const float *y, float *z, long long n) {
  for (long long i = 0; i < n; i++) z[i] = powf(x[i], y[i]);
}
