/* CPU oracle (test infrastructure only): the fp32 ops of the int8 Perch-family plan around the int8 GEMMs: the framed
 * log-mel front end (FE_LOGMEL), the im2col stem (STEM) on the fp32 GEMM (gemm_f32), the squeeze-excitation gate
 * (SE_GATE / SE), the spatial mean (MEAN) and the halo copy (PAD). Each lane of the reference's 4-lane NEON code is
 * an independent chain (frames, channels or output rows), so one scalar chain per lane restates it exactly. */
#define _DEFAULT_SOURCE /* M_PI */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static uint32_t fb(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float bf(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* log2_acc_f32x4 (src/gemm_f32.h:57-71): exponent split at sqrt(1/2), degree-8 polynomial in z = m - 1 */
float orc_log2_acc(float x) {
  const int32_t xi = (int32_t)fb(x);
  const int32_t t = (int32_t)((uint32_t)xi - 0x3f3504f3u);
  const int32_t e = t >> 23;
  const float z = bf((uint32_t)xi - ((uint32_t)e << 23)) - 1.f;
  float p = fmaf(z, 0.12125539f, -0.20643105f);
  p = fmaf(z, p, 0.21717128f);
  p = fmaf(z, p, -0.23910326f);
  p = fmaf(z, p, 0.28774428f);
  p = fmaf(z, p, -0.3606941f);
  p = fmaf(z, p, 0.4809185f);
  p = fmaf(z, p, -0.7213475f);
  p = fmaf(z, p, 1.4426949f);
  return fmaf(z, p, (float)e);
}

/* exp2_f32x4 (src/gemm_f32.h:74-85) */
float orc_exp2_f32(float t) {
  t = orc_fmin(orc_fmax(t, -126.f), 126.f);
  const float n = rintf(t), f = t - n;
  float p = 1.5403530e-4f;
  p = fmaf(p, f, 1.3333558e-3f);
  p = fmaf(p, f, 9.6181291e-3f);
  p = fmaf(p, f, 5.5504109e-2f);
  p = fmaf(p, f, 2.4022651e-1f);
  p = fmaf(p, f, 6.9314718e-1f);
  p = fmaf(p, f, 1.f);
  const int32_t ni = n != n ? 0 : (int32_t)n; /* FCVTZS of an integral value in [-126, 126] (NaN -> 0) */
  return bf(fb(p) + ((uint32_t)ni << 23));
}

/* sigmoid_f32x4 (src/gemm_f32.h:93-96) with rcp_f32x4 (:87-92): FRECPE and two Newton steps */
float orc_sigmoid_f32(float x) {
  const float d = 1.f + orc_exp2_f32(x * -1.44269504f);
  float r = orc_frecpe(d);
  r = r * orc_frecps(d, r);
  r = r * orc_frecps(d, r);
  return r;
}

/* ---------------------------------------------------------------- FE_LOGMEL (src/pc_kern_f32.c:28-149) */
static int bitrev(int i, int bits) { /* fft_bitrev (src/fft_tab.h:16-20) */
  int r = 0;
  for (int b = 0; b < bits; b++) r |= ((i >> b) & 1) << (bits - 1 - b);
  return r;
}

/* fft_dit_x4 (src/fft_tab.h:25-80) on one lane */
static void fft_dit(float *re, float *im, int M, const float *twr, const float *twi) {
  for (int i = 0; i < M; i += 4) {
    const float ar = re[i], ai = im[i], br = re[i + 1], bi = im[i + 1], cr = re[i + 2], ci = im[i + 2],
                dr = re[i + 3], di = im[i + 3];
    const float s0r = ar + br, s0i = ai + bi, d0r = ar - br, d0i = ai - bi;
    const float s1r = cr + dr, s1i = ci + di, d1r = cr - dr, d1i = ci - di;
    re[i] = s0r + s1r; im[i] = s0i + s1i;
    re[i + 2] = s0r - s1r; im[i + 2] = s0i - s1i;
    re[i + 1] = d0r + d1i; im[i + 1] = d0i - d1r;
    re[i + 3] = d0r - d1i; im[i + 3] = d0i + d1r;
  }
  int len = 8;
  for (; 2 * len <= M; len <<= 2) {
    const int h = len / 2, st1 = M / len, st2 = M / (2 * len);
    for (int i = 0; i < M; i += 2 * len)
      for (int j = 0; j < h; j++) {
        const float w1r = twr[j * st1], w1i = twi[j * st1], w2r = twr[j * st2], w2i = twi[j * st2];
        float *pr = re + i + j, *pi = im + i + j;
        const float ar = pr[0], ai = pi[0], br = pr[h], bi = pi[h], cr = pr[2 * h], ci = pi[2 * h], dr = pr[3 * h],
                    di = pi[3 * h];
        /* vfmsq_n_f32(vmulq_n_f32(b, w1r), bi, w1i) = b w1r - bi w1i with one fused step */
        float tr = fmaf(-bi, w1i, br * w1r), ti = fmaf(bi, w1r, br * w1i);
        const float a1r = ar + tr, a1i = ai + ti, b1r = ar - tr, b1i = ai - ti;
        tr = fmaf(-di, w1i, dr * w1r);
        ti = fmaf(di, w1r, dr * w1i);
        const float c1r = cr + tr, c1i = ci + ti, d1r = cr - tr, d1i = ci - ti;
        tr = fmaf(-c1i, w2i, c1r * w2r);
        ti = fmaf(c1i, w2r, c1r * w2i);
        pr[0] = a1r + tr; pi[0] = a1i + ti;
        pr[2 * h] = a1r - tr; pi[2 * h] = a1i - ti;
        const float ur = fmaf(-d1i, w2i, d1r * w2r), ui = fmaf(d1i, w2r, d1r * w2i);
        pr[h] = b1r + ui; pi[h] = b1i - ur;
        pr[3 * h] = b1r - ui; pi[3 * h] = b1i + ur;
      }
  }
  for (; len <= M; len <<= 1) {
    const int half = len / 2, step = M / len;
    for (int i = 0; i < M; i += len)
      for (int j = 0; j < half; j++) {
        const float wr = twr[j * step], wi = twi[j * step];
        const float xr = re[i + j + half], xi = im[i + j + half];
        const float vr = fmaf(-xi, wi, xr * wr), vi = fmaf(xi, wr, xr * wi);
        const float ur = re[i + j], ui = im[i + j];
        re[i + j] = ur + vr; im[i + j] = ui + vi;
        re[i + j + half] = ur - vr; im[i + j + half] = ui - vi;
      }
  }
}

/* the FFT on its own: M points of one lane in bit-reversed order, in place (for its order tests) */
void orc_fft_dit(float *re, float *im, int M, const float *twr, const float *twi) { fft_dit(re, im, M, twr, twi); }

int orc_logmel_frames(int nsamp, int frame, int hop, int pad) { return (nsamp + 2 * pad - frame) / hop + 1; }

int orc_logmel(const float *pcm, int nsamp, int frame, int hop, int pad, int nfft, int nmel, const float *window,
               const float *mel, float floor_, float scale, float *spec) {
  if (nfft < 16 || nfft > 2048 || (nfft & (nfft - 1)) || frame > nfft || hop <= 0 || pad < 0 || nmel < 1 || nmel > 512)
    return -1;
  const int M = nfft / 2, bins = nfft / 2 + 1, nfr = orc_logmel_frames(nsamp, frame, hop, pad);
  int lg = 0;
  while ((1 << lg) < M) lg++;
  int klo = bins, khi = 0;
  for (int j = 0; j < nmel; j++)
    for (int k = 0; k < bins; k++)
      if (mel[(size_t)j * bins + k] != 0.f) {
        if (k < klo) klo = k;
        if (k + 1 > khi) khi = k + 1;
      }
  if (khi == 0) klo = 0;
  float *win = calloc(nfft, sizeof(float)), *twr = malloc(sizeof(float) * M / 2), *twi = malloc(sizeof(float) * M / 2);
  float *pc = malloc(sizeof(float) * (khi + 1)), *ps = malloc(sizeof(float) * (khi + 1));
  float *re = malloc(sizeof(float) * M), *im = malloc(sizeof(float) * M), *mag = calloc(bins + 1, sizeof(float));
  memcpy(win, window, sizeof(float) * frame);
  for (int k = 0; k < M / 2; k++) { /* fft_twiddles (src/fft_tab.h:9-14) */
    double a = -2 * M_PI * k / M;
    twr[k] = (float)cos(a); twi[k] = (float)sin(a);
  }
  for (int k = 0; k < khi; k++) {
    double a = 2 * M_PI * k / nfft;
    pc[k] = (float)cos(a); ps[k] = (float)sin(a);
  }
  const int nz = (frame + 1) / 2;
  for (int t = 0; t < nfr; t++) {
    const long st = (long)t * hop - pad; /* the reference's padded signal y: pad zeros, pcm, zeros */
    for (int n = 0; n < M; n++) {
      const int r = bitrev(n, lg);
      if (n >= nz) { re[r] = 0.f; im[r] = 0.f; continue; }
      const long i0 = st + 2 * n, i1 = i0 + 1;
      const float y0 = i0 >= 0 && i0 < nsamp ? pcm[i0] : 0.f, y1 = i1 >= 0 && i1 < nsamp ? pcm[i1] : 0.f;
      re[r] = y0 * win[2 * n];
      im[r] = y1 * win[2 * n + 1];
    }
    fft_dit(re, im, M, twr, twi);
    for (int k = klo; k < khi; k++) {
      const int k2 = (k == 0 || k == M) ? 0 : M - k, ka = k == M ? 0 : k;
      const float Ar = re[ka], Ai = im[ka], Br = re[k2], Bi = -im[k2];
      const float Er = (Ar + Br) * 0.5f, Ei = (Ai + Bi) * 0.5f;
      const float Or = (Ai - Bi) * 0.5f, Oi = (Br - Ar) * 0.5f;
      const float c = pc[k], s = ps[k];
      const float Xr = fmaf(Oi, s, fmaf(Or, c, Er));
      const float Xi = fmaf(-Or, s, fmaf(Oi, c, Ei));
      mag[k] = sqrtf(fmaf(Xi, Xi, Xr * Xr));
    }
    for (int j = 0; j < nmel; j++) { /* the sparse mel rows in k order, alternating two accumulators */
      float a0 = 0.f, a1 = 0.f;
      int e = 0;
      for (int k = 0; k < bins; k++) {
        const float w = mel[(size_t)j * bins + k];
        if (w == 0.f) continue;
        if (e % 2 == 0) a0 = fmaf(mag[k], w, a0);
        else a1 = fmaf(mag[k], w, a1);
        e++;
      }
      spec[(size_t)t * nmel + j] = orc_log2_acc(orc_fmax(a0 + a1, floor_)) * 0.69314718f * scale;
    }
  }
  free(win); free(twr); free(twi); free(pc); free(ps); free(re); free(im); free(mag);
  return nfr;
}

/* ---------------------------------------------------------------- fp32 GEMM (src/gemm_f32.c) */
/* every row m < M and channel n < Np: one FMA chain over k < Kp from +0 (KB8X8F, src/gemm_f32_kblock.h), + b[n],
 * the activation (silu4_f32x4 / max 0), + residual, stored by out_row / the residual row rule (src/gemm_f32.c:40-57,
 * 78-131). w is the package layout [Np/8][Kp][8] (fp_pack, :22-35); gate (or NULL) scales A[m][k] first (fp32
 * multiply, gemm_f32_range_gate :167-193). A rows need Kp readable elements. */
void orc_gemm_f32(const float *A, int lda, int M, const float *w, const float *b, int Kp, int Np, const float *gate,
                  const orc_epi32 *e) {
  for (int m = 0; m < M; m++) {
    size_t orow = m;
    if (e->opad) orow = (size_t)((m / e->ow) + e->opad) * (e->ow + 2 * e->opad) + (m % e->ow) + e->opad;
    for (int n = 0; n < Np; n++) {
      float acc = 0.f;
      const float *wp = w + (size_t)(n / 8) * Kp * 8 + n % 8;
      for (int k = 0; k < Kp; k++) {
        float a = A[(size_t)m * lda + k];
        if (gate) a = a * gate[k];
        acc = fmaf(wp[(size_t)k * 8], a, acc);
      }
      float y = acc + b[n];
      if (e->act == 1) y = orc_silu_f32(y);
      else if (e->act == 2) y = orc_fmax(y, 0.f);
      if (e->res) {
        size_t rm = e->rpad ? (size_t)((m / e->rw) + e->rpad) * (e->rw + 2 * e->rpad) + m % e->rw + e->rpad : (size_t)m;
        y = y + e->res[rm * e->ldr + n];
      }
      e->out[orow * e->ldo + n] = y;
    }
  }
}

/* STEM (src/rt_ops_f32.c:416-425): pc_im2col1 (src/pc_kern_f32.c:150-161) then gemm_f32; a padded output has its
 * halo zeroed first */
void orc_stem_f32(const float *img, int H, int W, int k, int s, int Ho, int Wo, const float *w, const float *b, int Kp,
                  int Np, const orc_epi32 *e) {
  (void)H;
  const int M = Ho * Wo;
  float *col = calloc((size_t)M * Kp + 8, sizeof(float));
  for (int oy = 0; oy < Ho; oy++)
    for (int ox = 0; ox < Wo; ox++) {
      float *c = col + ((size_t)oy * Wo + ox) * Kp;
      int q = 0;
      for (int ky = 0; ky < k; ky++)
        for (int kx = 0; kx < k; kx++) c[q++] = img[(size_t)(oy * s + ky) * W + ox * s + kx];
    }
  if (e->opad) orc_zero_halo(e->out, Ho, Wo, e->ldo, e->opad, 4);
  orc_gemm_f32(col, Kp, M, w, b, Kp, Np, NULL, e);
  free(col);
}

/* ---------------------------------------------------------------- squeeze-excitation */
/* the gate of v24k32_se_fc1 + se_gate_range (src/v24_f32.c:164-179, src/rt_ops_f32.c:269-283): mean = chsum * (1/P);
 * fc1 with eight lane chains (two 4-lane accumulators over 8-channel steps) summed pairwise, + b1, SiLU by the C
 * library's expf (silu_s, src/v24_f32.c:160); fc2 from the bias, one FMA per row r; sigmoid_f32x4 */
/* the first FC of the SE gate (v24k32_se_fc1, src/v24_f32.c:164-179): per output r, eight lane chains over the
 * channels (two 4-lane accumulators over 8-channel steps: channel c feeds chain c % 8, a 4-channel tail the first
 * four), summed as ((a0 + a4) + (a1 + a5)) + ((a2 + a6) + (a3 + a7)) (vaddvq of a0 + a1), + b1, SiLU by the C
 * library's expf: s1 = x / (1 + expf(-x)). h16: the weights are rounded to fp16 first (SE_GATE16's fp16-held fc1) */
void orc_se_fc1(const float *mean, int C, int rd, const float *w1, int h16, const float *b1, float *s1) {
  for (int r = 0; r < rd; r++) {
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const float *w = w1 + (size_t)r * C;
    int c = 0;
    for (; c + 8 <= C; c += 8)
      for (int l = 0; l < 8; l++) a[l] = fmaf(h16 ? orc_h2f(orc_f2h(w[c + l])) : w[c + l], mean[c + l], a[l]);
    for (; c < C; c += 4)
      for (int l = 0; l < 4; l++) a[l] = fmaf(h16 ? orc_h2f(orc_f2h(w[c + l])) : w[c + l], mean[c + l], a[l]);
    const float v = ((a[0] + a[4]) + (a[1] + a[5])) + ((a[2] + a[6]) + (a[3] + a[7])); /* vaddvq(a0 + a1) */
    const float x = v + b1[r];
    s1[r] = x / (1.f + expf(-x));
  }
}

void orc_se_gate_f32(const float *chsum, int C, int rd, int P, const float *w1, const float *b1, const float *w2t,
                     const float *b2, float *gate) {
  float *mean = calloc(C, sizeof(float)), *s1 = calloc(rd, sizeof(float));
  const float inv = 1.f / (float)P;
  for (int c = 0; c < C; c++) mean[c] = chsum[c] * inv;
  orc_se_fc1(mean, C, rd, w1, 0, b1, s1);
  for (int c = 0; c < C; c++) {
    float g = b2[c];
    for (int r = 0; r < rd; r++) g = fmaf(w2t[(size_t)r * C + c], s1[r], g);
    gate[c] = orc_sigmoid_f32(g);
  }
  free(mean); free(s1);
}

/* SE in place (v24k32_se, src/v24_f32.c:181-210): D[p][c] *= gate[c] */
void orc_se_f32(float *D, int P, int C, const float *chsum, int rd, const float *w1, const float *b1, const float *w2t,
                const float *b2) {
  float *g = malloc(sizeof(float) * C);
  orc_se_gate_f32(chsum, C, rd, P, w1, b1, w2t, b2, g);
  for (int p = 0; p < P; p++)
    for (int c = 0; c < C; c++) D[(size_t)p * C + c] = D[(size_t)p * C + c] * g[c];
  free(g);
}

/* pc_mean_f32 (src/pc_kern_f32.c:342-348): a sum from +0 in p order, divided by (float)P */
void orc_mean_f32(const float *x, int P, int C, int ld, float *out) {
  for (int c = 0; c < C; c++) {
    float s = 0.f;
    for (int p = 0; p < P; p++) s = s + x[(size_t)p * ld + c];
    out[c] = s / (float)P;
  }
}

/* PAD (src/rt_ops_f32.c:503-508): zero halo, then the rows [H][W][ld] copied into [H+2h][W+2h][C] */
void orc_pad(const void *x, int H, int W, int C, int ld, int h, size_t esz, void *xp) {
  orc_zero_halo(xp, H, W, C, h, esz);
  for (int y = 0; y < H; y++)
    for (int xx = 0; xx < W; xx++)
      memcpy((char *)xp + ((size_t)(y + h) * (W + 2 * h) + xx + h) * C * esz, (const char *)x + ((size_t)y * W + xx) * ld * esz,
             esz * C);
}

/* the C library's expf elementwise (the reference's silu_s calls it; the checker of the device restatement) */
void orc_expf_n(const float *x, float *y, long long n) {
  for (long long i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* ---------------------------------------------------------------- fp16-path forms (variant 1) */
/* STEM with fp16 output (src/rt_ops_f16.c:167-180): the fp32 stem into [M][Np] rows, then channels < N rounded to
 * fp16 (vcvt_f16_f32, nearest even) into the padded output (pc_cvt_pad_f16, src/pc_kern_f16.c:104-113); the halo is
 * zeroed first, channels N..ldo untouched */
void orc_stem_f32to16(const float *img, int H, int W, int k, int s, int Ho, int Wo, const float *w, const float *b, int Kp,
                      int N, int Np, int act, uint16_t *out, int ldo, int opad) {
  float *tmp = calloc((size_t)Ho * Wo * Np + 8, sizeof(float));
  orc_epi32 e = {act, tmp, Np, 0, 0, NULL, 0, 0, 0};
  orc_stem_f32(img, H, W, k, s, Ho, Wo, w, b, Kp, Np, &e);
  if (opad) orc_zero_halo(out, Ho, Wo, ldo, opad, 2);
  for (int m = 0; m < Ho * Wo; m++) {
    uint16_t *o = out + ((size_t)(m / Wo + opad) * (Wo + 2 * opad) + m % Wo + opad) * ldo;
    for (int c = 0; c < N; c++) o[c] = orc_f2h(tmp[(size_t)m * Np + c]);
  }
  free(tmp);
}

/* SE fp16 (v24k16_se_gate + v24k16_se_scale, src/v24_fast.c:182-234): the fp32 gate of the fp32 SE with a sigmoid
 * that divides (sigm4: 1 / (1 + exp2_f32x4 value), IEEE division), rounded to fp16; D (fp16) multiplied by it in
 * fp16 */
void orc_se_f16(uint16_t *D, int P, int C, const float *chsum, int rd, const float *w1, const float *b1, const float *w2t,
                const float *b2) {
  float *mean = calloc(C, sizeof(float)), *s1 = calloc(rd, sizeof(float));
  uint16_t *g = malloc(sizeof(uint16_t) * C);
  const float inv = 1.f / (float)P;
  for (int c = 0; c < C; c++) mean[c] = chsum[c] * inv;
  orc_se_fc1(mean, C, rd, w1, 0, b1, s1);
  for (int c = 0; c < C; c++) {
    float v = b2[c];
    for (int r = 0; r < rd; r++) v = fmaf(w2t[(size_t)r * C + c], s1[r], v);
    g[c] = orc_f2h(1.f / (1.f + orc_exp2_f32(v * -1.44269504f)));
  }
  for (int p = 0; p < P; p++)
    for (int c = 0; c < C; c++) D[(size_t)p * C + c] = orc_h_mul(D[(size_t)p * C + c], g[c]);
  free(mean); free(s1); free(g);
}

/* pc_mean_f16 (src/pc_kern_f16.c:115-121): fp32 sums of the widened values from +0 in p order, divided by P */
void orc_mean_f16(const uint16_t *x, int P, int C, int ld, float *out) {
  for (int c = 0; c < C; c++) {
    float s = 0.f;
    for (int p = 0; p < P; p++) s = s + orc_h2f(x[(size_t)p * ld + c]);
    out[c] = s / (float)P;
  }
}

/* bnn_gemv_f32 / bnn_gemv_h16 (src/gemv.c:13-49): eight lane chains over k < K & ~7 (two 4-lane accumulators), the
 * K & ~3 remainder into the first, pairwise sum, then the scalar tail (product and sum rounded apart), + b, ReLU
 * as v < 0 ? 0 : v. w16 (or NULL) holds fp16 weights, else w32. */
void orc_gemv(const float *w32, const uint16_t *w16, const float *b, int N, int K, const float *x, int act, float *out) {
  const int K4 = K & ~3, K8 = K & ~7;
  for (int n = 0; n < N; n++) {
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int k = 0; k < K; k++) {
      const float wv = w16 ? orc_h2f(w16[(size_t)n * K + k]) : w32[(size_t)n * K + k];
      if (k < K8) a[k % 8] = fmaf(wv, x[k], a[k % 8]);
      else if (k < K4) a[k % 4] = fmaf(wv, x[k], a[k % 4]);
    }
    float s = ((a[0] + a[4]) + (a[1] + a[5])) + ((a[2] + a[6]) + (a[3] + a[7]));
    for (int k = K4; k < K; k++) {
      const float wv = w16 ? orc_h2f(w16[(size_t)n * K + k]) : w32[(size_t)n * K + k];
      s = s + wv * x[k];
    }
    const float v = s + b[n];
    out[n] = act == 2 && v < 0.f ? 0.f : v;
  }
}
