/* CPU oracle (test infrastructure only): the int8 prototype head of libbnneon (PROTO_S8). See oracle.h. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static inline uint32_t fbits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }

/* src/proto_s8n.c:28-51. Sum of squares in two 4-lane fused accumulators over 8-channel steps (lane j of the first
 * takes channels c + j, of the second c + 4 + j), reduced as ((t0 + t1) + (t2 + t3)) with t_j = s0_j + s1_j; max |x|
 * with FMAX (NaN-propagating) in the same lanes; q = FCVTAS(x * (127 / mx)) narrowed with saturation to int16, int8,
 * then floored at -127; zeros from C to Kp. */
void orc_quant_cells_f32(const float *x, int P, int C, int ld, float eps, int8_t *qa, int Kp, float *sx) {
  for (int p = 0; p < P; p++) {
    const float *r = x + (size_t)p * ld;
    float s0[4] = {0, 0, 0, 0}, s1[4] = {0, 0, 0, 0}, m0[4] = {0, 0, 0, 0}, m1[4] = {0, 0, 0, 0};
    for (int c = 0; c < C; c += 8)
      for (int j = 0; j < 4; j++) {
        float u0 = r[c + j], u1 = r[c + 4 + j];
        s0[j] = fmaf(u0, u0, s0[j]);
        s1[j] = fmaf(u1, u1, s1[j]);
        m0[j] = orc_fmax(m0[j], fabsf(u0));
        m1[j] = orc_fmax(m1[j], fabsf(u1));
      }
    float t[4], m[4];
    for (int j = 0; j < 4; j++) { t[j] = s0[j] + s1[j]; m[j] = orc_fmax(m0[j], m1[j]); }
    float den = sqrtf((t[0] + t[1]) + (t[2] + t[3])) + eps;
    float mx = orc_fmax(orc_fmax(m[0], m[1]), orc_fmax(m[2], m[3]));
    if (!(mx > 0)) mx = 1e-30f;
    sx[p] = mx / (127.f * den);
    const float inv = 127.f / mx;
    int8_t *q = qa + (size_t)p * Kp;
    for (int c = 0; c < C; c++) {
      int32_t v = orc_cvta_s32(r[c] * inv);
      int32_t h = v < -32768 ? -32768 : v > 32767 ? 32767 : v;   /* SQXTN to int16 */
      int32_t b = h < -128 ? -128 : h > 127 ? 127 : h;           /* SQXTN to int8 */
      q[c] = (int8_t)(b < -127 ? -127 : b);                       /* SMAX with -127 */
    }
    memset(q + C, 0, (size_t)(Kp - C));
  }
}

/* src/proto_s8n.c:115-132: the first n4-flagged panel with a lane of 4 weights (bytes l, l + 8 of two consecutive
 * 16-byte steps of one prototype) summing to more than 258 in |w|, or -1; -1 also when Kp % 32 (no n4 loop) */
int orc_proto_n4_check(const int8_t *qw, int Kp, const uint8_t *n4, int npanels) {
  if (Kp % 32) return -1;
  for (int pn = 0; pn < npanels; pn++) {
    if (!n4[pn]) continue;
    const int8_t *w = qw + (size_t)pn * Kp * 4;
    for (int k = 0; k < Kp; k += 32, w += 128)
      for (int ch = 0; ch < 4; ch++)
        for (int l = 0; l < 8; l++) {
          int s = abs(w[16 * ch + l]) + abs(w[16 * ch + l + 8]) + abs(w[64 + 16 * ch + l]) + abs(w[64 + 16 * ch + l + 8]);
          if (s > 258) return pn;
        }
  }
  return -1;
}

/* src/proto_s8n.c:139-164: colmax[j] = (max over cells p of (float)acc[p][j] * sx[p]) * sw[j] for every prototype
 * j < Np (the max starts from -inf and propagates NaN), exact int32 sums over Kp */
void orc_proto_colmax_s8n(const int8_t *qa, int Kp, const float *sx, int P, const int8_t *qw, const float *sw, int Np,
                          float *colmax) {
  const int kb = Kp / 16;
  for (int j = 0; j < Np; j++) {
    const int8_t *wp = qw + (size_t)(j / 4) * kb * 64 + (j % 4) * 16;
    float mx = -INFINITY;
    for (int p = 0; p < P; p++) {
      const int8_t *a = qa + (size_t)p * Kp;
      uint32_t acc = 0;
      for (int k = 0; k < Kp; k++) acc += (uint32_t)((int32_t)a[k] * (int32_t)wp[(size_t)(k / 16) * 64 + k % 16]);
      mx = orc_fmax(mx, (float)(int32_t)acc * sx[p]);
    }
    colmax[j] = mx * sw[j];
  }
}

/* src/pc_kern_f32.c:364-374: logit c = (sum over q < ppc of colmax * w, multiply then add, in order) + b; -2 when a
 * logit is not finite (|v| <= 3e38 fails) */
int orc_proto_logits(const float *colmax, const float *w, const float *b, int nc, int ppc, float *logits) {
  int bad = 0;
  for (int c = 0; c < nc; c++) {
    float s = 0;
    for (int q = 0; q < ppc; q++) {
      float t = colmax[(size_t)c * ppc + q] * w[(size_t)c * ppc + q];
      s = s + t;
    }
    float v = s + b[c];
    logits[c] = v;
    bad |= !(fabsf(v) <= 3.0e38f);
  }
  (void)fbits;
  return bad ? -2 : 0;
}

/* the PROTO_S8 op of one window (src/rt_ops_s8n.c:245-253) */
int orc_proto_s8(const float *x, int P, int C, int ld, float eps, int8_t *qa, int Kp, float *sx, const int8_t *qw,
                 const float *sw, int Np, float *colmax, const float *clsw, const float *clsb, int nc, int ppc,
                 float *logits) {
  orc_quant_cells_f32(x, P, C, ld, eps, qa, Kp, sx);
  orc_proto_colmax_s8n(qa, Kp, sx, P, qw, sw, Np, colmax);
  return orc_proto_logits(colmax, clsw, clsb, nc, ppc, logits);
}

/* src/pc_proto_s8.c:14-45 (pc_quant_cells_f16): the fp16 cells widened, the same sums and maxima as
 * orc_quant_cells_f32, q = FCVTAS(x * (127 / mx)) narrowed with saturation to int16 then int8 (no floor at -127);
 * rows [P][Kp], zeros from C */
void orc_quant_cells_f16(const uint16_t *x, int P, int C, int ld, float eps, int8_t *qa, int Kp, float *sx) {
  float *row = malloc(sizeof(float) * (size_t)C);
  for (int p = 0; p < P; p++) {
    const uint16_t *r = x + (size_t)p * ld;
    float s0[4] = {0, 0, 0, 0}, s1[4] = {0, 0, 0, 0}, m0[4] = {0, 0, 0, 0}, m1[4] = {0, 0, 0, 0};
    for (int c = 0; c < C; c++) row[c] = orc_h2f(r[c]);
    for (int c = 0; c < C; c += 8)
      for (int j = 0; j < 4; j++) {
        float u0 = row[c + j], u1 = row[c + 4 + j];
        s0[j] = fmaf(u0, u0, s0[j]);
        s1[j] = fmaf(u1, u1, s1[j]);
        m0[j] = orc_fmax(m0[j], fabsf(u0));
        m1[j] = orc_fmax(m1[j], fabsf(u1));
      }
    float t[4], m[4];
    for (int j = 0; j < 4; j++) { t[j] = s0[j] + s1[j]; m[j] = orc_fmax(m0[j], m1[j]); }
    float den = sqrtf((t[0] + t[1]) + (t[2] + t[3])) + eps;
    float mx = orc_fmax(orc_fmax(m[0], m[1]), orc_fmax(m[2], m[3]));
    if (!(mx > 0)) mx = 1e-30f;
    sx[p] = mx / (127.f * den);
    const float inv = 127.f / mx;
    int8_t *q = qa + (size_t)p * Kp;
    for (int c = 0; c < C; c++) {
      int32_t v = orc_cvta_s32(row[c] * inv);
      int32_t h = v < -32768 ? -32768 : v > 32767 ? 32767 : v;
      q[c] = (int8_t)(h < -128 ? -128 : h > 127 ? 127 : h);
    }
    memset(q + C, 0, (size_t)(Kp - C));
  }
  free(row);
}

/* src/pc_proto_s8.c:47-88 (pc_proto_colmax_s8): colmax[j] = (max over cells p, from -inf, FMAX, of
 * (float)acc[p][j] * sx[p]) * sw[j], the prototypes read from their panels qw [Np/12][K/4][12][4] */
void orc_proto_colmax_c12(const int8_t *qa, int Kp, const float *sx, int P, int K, const int8_t *qw, const float *sw,
                          int Np, float *colmax) {
  for (int j = 0; j < Np; j++) {
    float mx = -INFINITY;
    for (int p = 0; p < P; p++) {
      const int8_t *a = qa + (size_t)p * Kp;
      int32_t acc = 0;
      for (int k = 0; k < K; k++) acc += (int32_t)a[k] * (int32_t)qw[((size_t)(j / 12) * (K / 4) + k / 4) * 48 + (j % 12) * 4 + k % 4];
      mx = orc_fmax(mx, (float)acc * sx[p]);
    }
    colmax[j] = mx * sw[j];
  }
}

/* ---------------------------------------------------------------- fp32 / fp16 prototype heads (PROTO variants 0
 * and 1, PROTO_F32H) */

/* src/pc_kern_f32.c:350-362 (pc_l2norm_f32): per cell, the sum of squares in two 4-lane fused accumulators over
 * 8-channel steps reduced as ((t0 + t1) + (t2 + t3)), t_j = s0_j + s1_j (FADDP); den = sqrtf(sum) + eps; a = x / den
 * (IEEE division), rows [P][C] */
void orc_l2norm_f32(const float *x, int P, int C, int ld, float eps, float *a) {
  for (int p = 0; p < P; p++) {
    const float *r = x + (size_t)p * ld;
    float s0[4] = {0, 0, 0, 0}, s1[4] = {0, 0, 0, 0};
    for (int c = 0; c < C; c += 8)
      for (int j = 0; j < 4; j++) {
        s0[j] = fmaf(r[c + j], r[c + j], s0[j]);
        s1[j] = fmaf(r[c + 4 + j], r[c + 4 + j], s1[j]);
      }
    float t[4];
    for (int j = 0; j < 4; j++) t[j] = s0[j] + s1[j];
    const float den = sqrtf((t[0] + t[1]) + (t[2] + t[3])) + eps;
    for (int c = 0; c < C; c++) a[(size_t)p * C + c] = r[c] / den;
  }
}

/* src/pc_kern_f16.c:123-140 (pc_l2norm_f16): the same sums of the widened fp16 values; a = fp16(fp32(x) / den),
 * rounded to nearest even */
void orc_l2norm_f16(const uint16_t *x, int P, int C, int ld, float eps, uint16_t *a) {
  for (int p = 0; p < P; p++) {
    const uint16_t *r = x + (size_t)p * ld;
    float s0[4] = {0, 0, 0, 0}, s1[4] = {0, 0, 0, 0};
    for (int c = 0; c < C; c += 8)
      for (int j = 0; j < 4; j++) {
        const float u0 = orc_h2f(r[c + j]), u1 = orc_h2f(r[c + 4 + j]);
        s0[j] = fmaf(u0, u0, s0[j]);
        s1[j] = fmaf(u1, u1, s1[j]);
      }
    float t[4];
    for (int j = 0; j < 4; j++) t[j] = s0[j] + s1[j];
    const float den = sqrtf((t[0] + t[1]) + (t[2] + t[3])) + eps;
    for (int c = 0; c < C; c++) a[(size_t)p * C + c] = orc_f2h(orc_h2f(r[c]) / den);
  }
}

/* src/gemm_f32.c:443-460 (gemm_f32_colmax, the KB k-block of src/gemm_f32_kblock.h): colmax[n] = FMAX over rows m,
 * from -inf, of one fused chain from +0 over k < Kp in order of k; prototypes as fp32 panels [Np/8][Kp][8] */
void orc_colmax_f32(const float *A, int lda, int M, const float *wp, int Kp, int Np, float *colmax) {
  for (int n = 0; n < Np; n++) {
    const float *w = wp + (size_t)(n / 8) * Kp * 8 + n % 8;
    float mx = -INFINITY;
    for (int m = 0; m < M; m++) {
      float acc = 0.f;
      for (int k = 0; k < Kp; k++) acc = fmaf(w[(size_t)k * 8], A[(size_t)m * lda + k], acc);
      mx = orc_fmax(mx, acc);
    }
    colmax[n] = mx;
  }
}

/* src/pc_kern_f32.c:378-407 (pc_proto_colmax_f32h): as orc_colmax_f32 with the prototypes stored in fp16 panels
 * [Np/8][K][8], each weight widened exactly (FCVTL) before its fused multiply-add; cells a [P][K] */
void orc_colmax_f32h(const float *a, int P, int K, const uint16_t *w16, int Np, float *colmax) {
  for (int n = 0; n < Np; n++) {
    const uint16_t *w = w16 + (size_t)(n / 8) * K * 8 + n % 8;
    float mx = -INFINITY;
    for (int p = 0; p < P; p++) {
      float acc = 0.f;
      for (int k = 0; k < K; k++) acc = fmaf(orc_h2f(w[(size_t)k * 8]), a[(size_t)p * K + k], acc);
      mx = orc_fmax(mx, acc);
    }
    colmax[n] = mx;
  }
}

/* K blocks of the fp16 GEMM (kblocks, src/gemm_f16.c:55-58) */
static void f16_kblocks(int Kp, int *nblk, int *bs) {
  *nblk = (Kp + 127) / 128;
  *bs = ((Kp + *nblk - 1) / *nblk + 7) & ~7;
}

/* src/gemm_f16.c:210-253 (gemm_f16_colmax_range over every panel): per output and K block, an fp16 fused chain from
 * +0 over the block's k in order; one block: the chain widened; several: an fp32 sum from +0 of the widened chains
 * in block order. colmax[n] = FMAX over rows, from -inf. Prototypes as hpack panels [Np/16][Kp][16], then a tail
 * panel [Kp][8] when Np % 16 == 8 */
void orc_colmax_f16(const uint16_t *A, int lda, int M, const uint16_t *W, int Kp, int Np, float *colmax) {
  int nblk, bs;
  f16_kblocks(Kp, &nblk, &bs);
  const int n16 = Np / 16;
  for (int n = 0; n < Np; n++) {
    const int pan = n / 16, wide = pan < n16, ws = wide ? 16 : 8;
    const uint16_t *w = W + (size_t)pan * Kp * 16 + (wide ? n % 16 : n - 16 * n16);
    float mx = -INFINITY;
    for (int m = 0; m < M; m++) {
      float fb = 0.f, v = 0.f;
      for (int kb = 0; kb < Kp; kb += bs) {
        const int kn = Kp - kb < bs ? Kp - kb : bs;
        uint16_t acc = 0;
        for (int k = kb; k < kb + kn; k++) acc = orc_h_fma(w[(size_t)k * ws], A[(size_t)m * lda + k], acc);
        if (nblk > 1) fb = fb + orc_h2f(acc);
        else v = orc_h2f(acc);
      }
      mx = orc_fmax(mx, nblk > 1 ? fb : v);
    }
    colmax[n] = mx;
  }
}

/* PROTO variant 0 of one window (proto_run, src/rt_ops_f32.c:563-570): cells x [P][ld] -> scratch a [P][C],
 * colmax [Np], logits [nc]; returns orc_proto_logits' code */
int orc_proto_f32(const float *x, int P, int C, int ld, float eps, float *a, const float *wp, int Np, float *colmax,
                  const float *clsw, const float *clsb, int nc, int ppc, float *logits) {
  orc_l2norm_f32(x, P, C, ld, eps, a);
  orc_colmax_f32(a, C, P, wp, C, Np, colmax);
  return orc_proto_logits(colmax, clsw, clsb, nc, ppc, logits);
}

/* PROTO_F32H of one window (proto_h_run, src/rt_ops_f32.c:583-590) */
int orc_proto_f32h(const float *x, int P, int C, int ld, float eps, float *a, const uint16_t *w16, int Np,
                   float *colmax, const float *clsw, const float *clsb, int nc, int ppc, float *logits) {
  orc_l2norm_f32(x, P, C, ld, eps, a);
  orc_colmax_f32h(a, P, C, w16, Np, colmax);
  return orc_proto_logits(colmax, clsw, clsb, nc, ppc, logits);
}

/* PROTO variant 1 of one window (proto_run, src/rt_ops_f16.c:236-250): fp16 cells, fp16 scratch a [P][C] */
int orc_proto_f16(const uint16_t *x, int P, int C, int ld, float eps, uint16_t *a, const uint16_t *W, int Np,
                  float *colmax, const float *clsw, const float *clsb, int nc, int ppc, float *logits) {
  orc_l2norm_f16(x, P, C, ld, eps, a);
  orc_colmax_f16(a, C, P, W, C, Np, colmax);
  return orc_proto_logits(colmax, clsw, clsb, nc, ppc, logits);
}
