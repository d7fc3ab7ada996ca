/* CPU oracle (test infrastructure only): libbnneon's fp16 GEMM (src/gemm_f16.c:49-171, the PW f16 op of
 * src/rt_ops_f16.c:53-81). See oracle.h. fp16 values are bit patterns; arithmetic through orc_h_* (dw.c). */
#include <math.h>
#include <string.h>

#include "oracle.h"

/* fp32 -> fp16, round to nearest even, denormals kept, overflow to infinity (FCVT h, s with FPCR defaults) */
uint16_t orc_f2h(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
  const uint32_t e = (u >> 23) & 0xff, m = u & 0x7fffff;
  if (e == 0xff) return (uint16_t)(sign | (m ? 0x7e00 : 0x7c00));
  if (e == 0 && m == 0) return sign;
  /* value = M * 2^E exactly, M < 2^24 */
  const uint32_t M = e ? (m | 0x800000) : m;
  const int E = e ? (int)e - 150 : -149;
  /* target: fp16 quantum 2^max(exponent - 10, -24) */
  int L = 0;
  for (uint32_t t = M; t; t >>= 1) L++;
  int er = E + L - 11;
  if (er < -24) er = -24;
  const int sh = er - E;
  uint32_t q;
  if (sh <= 0) q = M << (-sh);
  else if (sh >= 32) q = 0;
  else {
    q = M >> sh;
    const uint32_t r = M & ((1u << sh) - 1), half = 1u << (sh - 1);
    if (r > half || (r == half && (q & 1))) q++;
  }
  if (q >= 2048) { q >>= 1; er++; }
  if (q < 1024) return (uint16_t)(sign | q);          /* denormal (er == -24) or zero */
  const int ef = er + 25;
  if (ef >= 31) return (uint16_t)(sign | 0x7c00);
  return (uint16_t)(sign | (ef << 10) | (q - 1024));
}

/* K blocks of gemm_f16 (kblocks, src/gemm_f16.c:55-58): as few as possible with <= 128 k-steps, balanced, multiples
 * of 8 */
static void kblocks(int Kp, int *nblk, int *bs) {
  *nblk = (Kp + 127) / 128;
  *bs = ((Kp + *nblk - 1) / *nblk + 7) & ~7;
}

void orc_gemm_f16(const uint16_t *A, int lda, int M, const uint16_t *W, int N, int Kp, const float *b32,
                  const uint16_t *b16, const orc_epi16 *e) {
  int nblk, bs;
  kblocks(Kp, &nblk, &bs);
  for (int m = 0; m < M; m++) {
    size_t orow = (size_t)m;
    if (e->opad) orow = (size_t)((m / e->ow) + e->opad) * (e->ow + 2 * e->opad) + (m % e->ow) + e->opad;
    for (int n = 0; n < e->ldo && n < ((N + 7) & ~7); n++) {
      uint16_t v;  /* pad channels n >= N: zero weights and bias */
      float fb = 0.f;
      uint16_t acc = 0;
      for (int kb = 0; kb < Kp; kb += bs) {
        const int kn = Kp - kb < bs ? Kp - kb : bs;
        acc = 0;
        for (int k = kb; k < kb + kn; k++)
          acc = orc_h_fma(n < N ? W[(size_t)n * Kp + k] : 0, A[(size_t)m * lda + k], acc);
        if (nblk > 1) fb = fb + orc_h2f(acc);
      }
      if (nblk > 1) v = orc_f2h(fb + (n < N ? b32[n] : 0.f));
      else v = orc_h_add(acc, n < N ? b16[n] : 0);
      if (e->act == 1) v = orc_silu_lut_h(v);
      else if (e->act == 2) v = orc_h_max(v, 0);
      if (e->res) v = orc_h_add(v, e->res[(size_t)m * e->ldr + n]);
      e->out[orow * e->ldo + n] = v;
    }
  }
}
