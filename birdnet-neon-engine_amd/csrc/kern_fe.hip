// Framed log-mel front end (libbnneon's FE_LOGMEL, pc_logmel_new / pc_logmel_run, src/pc_kern_f32.c:28-149) on gfx950,
// bit-identical: the same radix-2 decimation-in-time FFT of nfft/2 complex points (two real samples per point, the
// first two levels fused, then radix-2^2 passes, then a last radix-2 level when the level count is odd;
// src/fft_tab.h:25-80), the same real-input split, magnitudes, sparse mel sums in two alternating accumulators,
// log2_acc polynomial and scale. Every reference lane is one frame; here one block transforms FPB frames of one
// window in LDS, each butterfly a work item, with the reference's operations in its order per element.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "bnh_internal.h"
#include "bnh_num.h"

struct bnh_logmel {
  int nsamp, frame, hop, pad, nfft, M, lg, nmel, nfr, klo, khi, nnz;
  float floor_, scale;
  float *win;         // [nfft], zero past the frame
  float *twr, *twi;   // e^{-2 pi i k / M}, k < M / 2
  float *pc, *ps;     // cos, sin (2 pi k / nfft), k < khi
  int *mel_off;       // [nmel + 1]
  int *mel_k;         // [nnz]
  float *mel_w;       // [nnz]
};

#define FE_FPB 4  // frames per block (the frame index of a flat item is three comparisons)
static_assert(FE_FPB == 4, "k_logmel finds a flat item's frame with three comparisons");

// log2_acc_f32x4 (src/gemm_f32.h:57-71) on one lane
__device__ __forceinline__ float fe_log2_acc(float x) {
  const int32_t xi = (int32_t)__float_as_uint(x);
  const int32_t e = (int32_t)((uint32_t)xi - 0x3f3504f3u) >> 23;
  const float z = __uint_as_float((uint32_t)xi - ((uint32_t)e << 23)) - 1.f;
  float p = __builtin_fmaf(z, 0.12125539f, -0.20643105f);
  p = __builtin_fmaf(z, p, 0.21717128f);
  p = __builtin_fmaf(z, p, -0.23910326f);
  p = __builtin_fmaf(z, p, 0.28774428f);
  p = __builtin_fmaf(z, p, -0.3606941f);
  p = __builtin_fmaf(z, p, 0.4809185f);
  p = __builtin_fmaf(z, p, -0.7213475f);
  p = __builtin_fmaf(z, p, 1.4426949f);
  return __builtin_fmaf(z, p, (float)e);
}

// b w_r - bi w_i and b w_i + bi w_r with the reference's one fused step each (vfmsq_n / vfmaq_n on a product)
__device__ __forceinline__ void fe_cmul(float br, float bi, float wr, float wi, float &tr, float &ti) {
  tr = __builtin_fmaf(-bi, wi, br * wr);
  ti = __builtin_fmaf(bi, wr, br * wi);
}

// grid (ceil(nfr / FPB), B); dynamic LDS: re, im [FPB][M], mag [FPB][bins] and the twiddles (cos, sin [M / 2]: read
// by every frame and pass, staged once per block)
__global__ __launch_bounds__(256) void k_logmel(const float *__restrict__ pcm, long long p_ws, float *__restrict__ spec,
                                                long long s_ws, bnh_logmel F) {
  extern __shared__ float lds[];
  const int M = F.M, bins = M + 1, tid = threadIdx.x;
  float *re = lds, *im = lds + FE_FPB * M, *mag = lds + 2 * FE_FPB * M;
  float *twr = mag + FE_FPB * bins, *twi = twr + M / 2;
  for (int i = tid; i < M / 2; i += 256) {
    twr[i] = F.twr[i];
    twi[i] = F.twi[i];
  }
  const int t0 = blockIdx.x * FE_FPB, win = blockIdx.y;
  const float *x = pcm + win * p_ws;
  const int nz = (F.frame + 1) / 2;
  // M = 2^lg (lg >= 3): every index split of the FFT passes is a shift and a mask, not an integer division
  const int lg = F.lg;
  // z[n] = w[2n] y[2n] + i w[2n+1] y[2n+1], stored at the bit-reversed position
  for (int it = tid; it < FE_FPB * M; it += 256) {
    const int f = it >> lg, n = it & (M - 1);
    const int t = t0 + f < F.nfr ? t0 + f : F.nfr - 1;
    const int r = (int)(__builtin_bitreverse32((uint32_t)n) >> (32 - F.lg));
    float vr = 0.f, vi = 0.f;
    if (n < nz) {
      const long long i0 = (long long)t * F.hop - F.pad + 2 * n, i1 = i0 + 1;
      const float y0 = i0 >= 0 && i0 < F.nsamp ? x[i0] : 0.f, y1 = i1 >= 0 && i1 < F.nsamp ? x[i1] : 0.f;
      vr = y0 * F.win[2 * n];
      vi = y1 * F.win[2 * n + 1];
    }
    re[f * M + r] = vr;
    im[f * M + r] = vi;
  }
  __syncthreads();
  // levels 1 and 2 fused, no twiddles
  for (int it = tid; it < FE_FPB * (M / 4); it += 256) {
    const int f = it >> (lg - 2), i = 4 * (it & (M / 4 - 1));
    float *pr = re + f * M + i, *pi = im + f * M + i;
    const float ar = pr[0], ai = pi[0], br = pr[1], bi = pi[1], cr = pr[2], ci = pi[2], dr = pr[3], di = pi[3];
    const float s0r = ar + br, s0i = ai + bi, d0r = ar - br, d0i = ai - bi;
    const float s1r = cr + dr, s1i = ci + di, d1r = cr - dr, d1i = ci - di;
    pr[0] = s0r + s1r; pi[0] = s0i + s1i;
    pr[2] = s0r - s1r; pi[2] = s0i - s1i;
    pr[1] = d0r + d1i; pi[1] = d0i - d1r;
    pr[3] = d0r - d1i; pi[3] = d0i + d1r;
  }
  int len = 8, lgl = 3;
  for (; 2 * len <= M; len <<= 2, lgl += 2) {  // radix-2^2 passes: levels len and 2 len
    __syncthreads();
    const int h = len / 2, st1 = M / len, st2 = M / (2 * len);
    for (int it = tid; it < FE_FPB * (M / 4); it += 256) {
      const int f = it >> (lg - 2), g = it & (M / 4 - 1), j = g & (h - 1), i = (g >> (lgl - 1)) << (lgl + 1);
      const float w1r = twr[j * st1], w1i = twi[j * st1], w2r = twr[j * st2], w2i = twi[j * st2];
      float *pr = re + f * M + i + j, *pi = im + f * M + i + j;
      const float ar = pr[0], ai = pi[0], br = pr[h], bi = pi[h], cr = pr[2 * h], ci = pi[2 * h], dr = pr[3 * h],
                  di = pi[3 * h];
      float tr, ti;
      fe_cmul(br, bi, w1r, w1i, tr, ti);
      const float a1r = ar + tr, a1i = ai + ti, b1r = ar - tr, b1i = ai - ti;
      fe_cmul(dr, di, w1r, w1i, tr, ti);
      const float c1r = cr + tr, c1i = ci + ti, d1r = cr - tr, d1i = ci - ti;
      fe_cmul(c1r, c1i, w2r, w2i, tr, ti);
      pr[0] = a1r + tr; pi[0] = a1i + ti;
      pr[2 * h] = a1r - tr; pi[2 * h] = a1i - ti;
      float ur, ui;
      fe_cmul(d1r, d1i, w2r, w2i, ur, ui);
      pr[h] = b1r + ui; pi[h] = b1i - ur;
      pr[3 * h] = b1r - ui; pi[3 * h] = b1i + ur;
    }
  }
  for (; len <= M; len <<= 1, lgl++) {  // a last single level
    __syncthreads();
    const int half = len / 2, step = M / len;
    for (int it = tid; it < FE_FPB * (M / 2); it += 256) {
      const int f = it >> (lg - 1), g = it & (M / 2 - 1), j = g & (half - 1), i = (g >> (lgl - 1)) << lgl;
      const float wr = twr[j * step], wi = twi[j * step];
      float *pr = re + f * M + i + j, *pi = im + f * M + i + j;
      float vr, vi;
      fe_cmul(pr[half], pi[half], wr, wi, vr, vi);
      const float ur = pr[0], ui = pi[0];
      pr[0] = ur + vr; pi[0] = ui + vi;
      pr[half] = ur - vr; pi[half] = ui - vi;
    }
  }
  __syncthreads();
  // real-input split and magnitudes of bins [klo, khi)
  const int nk = F.khi - F.klo;
  for (int it = tid; it < FE_FPB * nk; it += 256) {
    const int f = (it >= nk) + (it >= 2 * nk) + (it >= 3 * nk), k = F.klo + it - f * nk;  // FPB 4 frames
    const int k2 = (k == 0 || k == M) ? 0 : M - k, ka = k == M ? 0 : k;
    const float *fr = re + f * M, *fi = im + f * M;
    const float Ar = fr[ka], Ai = fi[ka], Br = fr[k2], Bi = -fi[k2];
    const float Er = (Ar + Br) * 0.5f, Ei = (Ai + Bi) * 0.5f;
    const float Or = (Ai - Bi) * 0.5f, Oi = (Br - Ar) * 0.5f;
    const float c = F.pc[k], s = F.ps[k];
    const float Xr = __builtin_fmaf(Oi, s, __builtin_fmaf(Or, c, Er));
    const float Xi = __builtin_fmaf(-Or, s, __builtin_fmaf(Oi, c, Ei));
    mag[f * bins + k] = __builtin_sqrtf(__builtin_fmaf(Xi, Xi, Xr * Xr));
  }
  __syncthreads();
  for (int it = tid; it < FE_FPB * F.nmel; it += 256) {
    const int f = (it >= F.nmel) + (it >= 2 * F.nmel) + (it >= 3 * F.nmel), j = it - f * F.nmel, t = t0 + f;
    if (t >= F.nfr) continue;
    float a0 = 0.f, a1 = 0.f;
    const int e0 = F.mel_off[j], e1 = F.mel_off[j + 1];
    int e = e0;
    for (; e + 2 <= e1; e += 2) {
      a0 = __builtin_fmaf(mag[f * bins + F.mel_k[e]], F.mel_w[e], a0);
      a1 = __builtin_fmaf(mag[f * bins + F.mel_k[e + 1]], F.mel_w[e + 1], a1);
    }
    if (e < e1) a0 = __builtin_fmaf(mag[f * bins + F.mel_k[e]], F.mel_w[e], a0);
    const float v = fe_log2_acc(bnh_fmax(a0 + a1, F.floor_)) * 0.69314718f * F.scale;
    spec[win * s_ws + (long long)t * F.nmel + j] = v;
  }
}

extern "C" {

bnh_logmel *bnh_logmel_new(int nsamp, int frame, int hop, int pad, int nfft, int nmel, const float *window,
                           const float *mel, float floor_, float scale) {
  if (nfft < 16 || nfft > 2048 || (nfft & (nfft - 1)) || frame > nfft || frame < 1 || hop <= 0 || pad < 0 ||
      nmel < 1 || nmel > 512 || nsamp + 2 * pad < frame || !window || !mel) {
    bnh_fail("bnh_logmel_new: nfft %d frame %d hop %d pad %d nmel %d nsamp %d: expected nfft a power of two in "
             "16..2048, 1 <= frame <= nfft, hop > 0, pad >= 0, 1..512 mel bins, at least one frame, and both tensors",
             nfft, frame, hop, pad, nmel, nsamp);
    return nullptr;
  }
  bnh_logmel *F = (bnh_logmel *)calloc(1, sizeof *F);
  if (!F) { bnh_fail("bnh_logmel_new: out of host memory"); return nullptr; }
  F->nsamp = nsamp; F->frame = frame; F->hop = hop; F->pad = pad; F->nfft = nfft; F->M = nfft / 2; F->nmel = nmel;
  F->nfr = (nsamp + 2 * pad - frame) / hop + 1;
  while ((1 << F->lg) < F->M) F->lg++;
  F->floor_ = floor_; F->scale = scale;
  const int bins = nfft / 2 + 1, M = F->M;
  F->klo = bins; F->khi = 0;
  int nnz = 0;
  for (int j = 0; j < nmel; j++)
    for (int k = 0; k < bins; k++)
      if (mel[(size_t)j * bins + k] != 0.f) {
        nnz++;
        if (k < F->klo) F->klo = k;
        if (k + 1 > F->khi) F->khi = k + 1;
      }
  if (F->khi == 0) F->klo = 0;
  F->nnz = nnz;
  float *win = (float *)calloc(nfft, 4), *tw = (float *)malloc(4 * (size_t)M), *pcs = (float *)malloc(8 * (size_t)(F->khi + 1));
  int *off = (int *)malloc(4 * (size_t)(nmel + 1)), *mk = (int *)malloc(4 * (size_t)(nnz + 1));
  float *mw = (float *)malloc(4 * (size_t)(nnz + 1));
  bool ok = win && tw && pcs && off && mk && mw;
  if (ok) {
    memcpy(win, window, 4 * (size_t)frame);
    for (int k = 0; k < M / 2; k++) {  // fft_twiddles (src/fft_tab.h:9-14): double, rounded once
      const double a = -2 * M_PI * k / M;
      tw[k] = (float)cos(a);
      tw[M / 2 + k] = (float)sin(a);
    }
    for (int k = 0; k < F->khi; k++) {
      const double a = 2 * M_PI * k / nfft;
      pcs[k] = (float)cos(a);
      pcs[F->khi + 1 + k] = (float)sin(a);
    }
    nnz = 0;
    for (int j = 0; j < nmel; j++) {
      off[j] = nnz;
      for (int k = 0; k < bins; k++)
        if (mel[(size_t)j * bins + k] != 0.f) { mk[nnz] = k; mw[nnz] = mel[(size_t)j * bins + k]; nnz++; }
    }
    off[nmel] = nnz;
    ok = (F->win = (float *)bnh_malloc(4 * (size_t)nfft)) && (F->twr = (float *)bnh_malloc(4 * (size_t)M)) &&
         (F->pc = (float *)bnh_malloc(8 * (size_t)(F->khi + 1))) && (F->mel_off = (int *)bnh_malloc(4 * (size_t)(nmel + 1))) &&
         (F->mel_k = (int *)bnh_malloc(4 * (size_t)(nnz + 1))) && (F->mel_w = (float *)bnh_malloc(4 * (size_t)(nnz + 1))) &&
         !bnh_memcpy_h2d(F->win, win, 4 * (size_t)nfft) && !bnh_memcpy_h2d(F->twr, tw, 4 * (size_t)M) &&
         !bnh_memcpy_h2d(F->pc, pcs, 8 * (size_t)(F->khi + 1)) && !bnh_memcpy_h2d(F->mel_off, off, 4 * (size_t)(nmel + 1)) &&
         !bnh_memcpy_h2d(F->mel_k, mk, 4 * (size_t)(nnz + 1)) && !bnh_memcpy_h2d(F->mel_w, mw, 4 * (size_t)(nnz + 1));
    if (ok) {
      F->twi = F->twr + M / 2;
      F->ps = F->pc + F->khi + 1;
    }
  } else {
    bnh_fail("bnh_logmel_new: out of host memory");
  }
  free(win); free(tw); free(pcs); free(off); free(mk); free(mw);
  if (!ok) { bnh_logmel_free(F); return nullptr; }
  return F;
}

void bnh_logmel_free(bnh_logmel *F) {
  if (!F) return;
  bnh_free(F->win); bnh_free(F->twr); bnh_free(F->pc); bnh_free(F->mel_off); bnh_free(F->mel_k); bnh_free(F->mel_w);
  free(F);
}

int bnh_logmel_frames(const bnh_logmel *F) { return F ? F->nfr : -1; }

int bnh_logmel_run(const bnh_logmel *F, const float *pcm, long long p_ws, float *spec, long long s_ws, int B,
               void *stream) {
  BNH_REQ(F && pcm && spec && B > 0);
  BNH_REQ(B == 1 || (p_ws >= F->nsamp && s_ws >= (long long)F->nfr * F->nmel));
  const size_t lds = sizeof(float) * (FE_FPB * (2 * (size_t)F->M + F->M + 1) + F->M);
  BNH_REQ(lds <= 64 * 1024);  // nfft <= 2048: at most 53 KB
  hipLaunchKernelGGL(k_logmel, dim3((unsigned)bnh_ceil_div(F->nfr, FE_FPB), (unsigned)B), dim3(256), lds,
                     bnh_stream(stream), pcm, p_ws, spec, s_ws, *F);
  BNH_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
